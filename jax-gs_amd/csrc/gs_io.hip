// PLY vertex records of the Gaussians, packed and unpacked on gfx950.
//
// Reference: jax_gs/io/ply.py:6-123.  A vertex is 62 little-endian float32 values:
//   x y z | nx ny nz (0) | f_dc_0..2 = sh[0][c] | f_rest_i = sh[1 + i / 3][i % 3], i < 45
//   | opacity | scale_0..2 | rot_0..3
// (coefficient-major, channel-minor: the reference's f_rest is sh[:, 1:, :].reshape(-1, 45),
// unlike the INRIA viewer's channel-major layout).  Packing the records on the device
// turns a checkpoint into one contiguous copy to the host; one thread writes one value
// of the [N, 62] record array (consecutive threads, consecutive bytes) and reads it from
// its parameter array, and unpacking is the same map read the other way.
#include "gs_common.h"

namespace gs {
namespace {

constexpr int kPlyFloats = 62;

// Parameter array and offset of record value j: 0 means, 1 normals (zero), 2 sh,
// 3 opacity, 4 scales, 5 quaternions.
__device__ inline void ply_field(int j, int& arr, int& off) {
  if (j < 3) { arr = 0; off = j; }
  else if (j < 6) { arr = 1; off = 0; }
  else if (j < 54) { arr = 2; off = j - 6; }  // sh[k][c] at k * 3 + c: f_dc then f_rest
  else if (j == 54) { arr = 3; off = 0; }
  else if (j < 58) { arr = 4; off = j - 55; }
  else { arr = 5; off = j - 58; }
}

template <bool PACK>
__global__ __launch_bounds__(256) void ply_kernel(int64_t n, float* __restrict__ means, float* __restrict__ scales,
                                                  float* __restrict__ quats, float* __restrict__ opac,
                                                  float* __restrict__ sh, float* __restrict__ rec) {
  const int64_t total = n * kPlyFloats;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
    const int64_t v = t < 0x7fffffff ? (int64_t)((uint32_t)t / (uint32_t)kPlyFloats) : t / kPlyFloats;
    const int j = (int)(t - v * kPlyFloats);
    int arr, off;
    ply_field(j, arr, off);
    float* p = nullptr;
    switch (arr) {
      case 0: p = means + v * 3 + off; break;
      case 2: p = sh + v * 48 + off; break;
      case 3: p = opac + v; break;
      case 4: p = scales + v * 3 + off; break;
      case 5: p = quats + v * 4 + off; break;
      default: break;
    }
    if (PACK) rec[t] = p ? *p : 0.0f;
    else if (p) *p = rec[t];
  }
}

}  // namespace
}  // namespace gs

using namespace gs;

template <bool PACK>
static int ply_launch(const char* name, void* stream, int64_t n, int sh_k, float* means, float* scales, float* quats,
                      float* opac, float* sh, float* records) {
  GS_REQUIRE(n >= 0, "%s: n out of range", name);
  GS_REQUIRE(sh_k == 16, "%s: the PLY layout holds degree-3 SH (16 coefficients), got %d", name, sh_k);
  GS_REQUIRE(n == 0 || (means && scales && quats && opac && sh && records), "%s: NULL argument", name);
  if (n == 0) return GS_OK;
  const int64_t total = n * kPlyFloats;
  const int blocks = (int)std::min<int64_t>(div_up(total, 256), 65536);
  hipLaunchKernelGGL(ply_kernel<PACK>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, n, means, scales, quats, opac,
                     sh, records);
  GS_LAUNCH_CHECK(name);
  return GS_OK;
}

extern "C" int gs_ply_pack(void* stream, int64_t n, int sh_k, const float* means, const float* scales,
                           const float* quats, const float* opacities, const float* sh_coeffs, float* records) {
  return ply_launch<true>("gs_ply_pack", stream, n, sh_k, const_cast<float*>(means), const_cast<float*>(scales),
                          const_cast<float*>(quats), const_cast<float*>(opacities), const_cast<float*>(sh_coeffs),
                          records);
}

extern "C" int gs_ply_unpack(void* stream, int64_t n, int sh_k, const float* records, float* means, float* scales,
                             float* quats, float* opacities, float* sh_coeffs) {
  return ply_launch<false>("gs_ply_unpack", stream, n, sh_k, means, scales, quats, opacities, sh_coeffs,
                           const_cast<float*>(records));
}
