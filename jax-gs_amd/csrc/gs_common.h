// Shared device helpers for the gfx950 rasterizer kernels.
//
// Build contract: every translation unit is compiled with -ffp-contract=off so that
// the per-Gaussian arithmetic (projection, covariance, radius, tile rectangle, depth
// key) rounds exactly like its sequential float32 statement; kernels that want fused
// multiply-adds call fmaf() explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gs_raster.h"

namespace gs {

constexpr int kTile = GS_TILE_SIZE;                 // rasterizer.py:6
constexpr int kOffset = GS_OFFSET_SIZE;             // rasterizer.py:7
constexpr int kBlock = GS_BLOCK_SIZE;               // rasterizer.py:8
constexpr int kMaxTileEntries = GS_MAX_TILE_INTERACTIONS;  // rasterizer.py:10
constexpr int kRec = GS_REC_STRIDE;
constexpr int kDepthBits = 13;                      // rasterizer.py:84
// The depth quantum is bits(z) >> 18 with an arithmetic shift (rasterizer.py:94-95), a
// signed 14-bit value in [-8192, 8191]; sort keys hold it plus 8192, so that the
// quanta of negative depths (which the reference sorts first) come first.
constexpr int kDepthKeyBias = 8192;
constexpr int kDepthKeyBits = 14;
constexpr int kDepthBinEmpty = 1 << kDepthKeyBits;  // Gaussians with no tile
__host__ __device__ inline uint32_t depth_key(uint32_t depth_bits) {
  return (uint32_t)(((int32_t)depth_bits >> (31 - kDepthBits)) + kDepthKeyBias);
}

// exp(x) in float32 from Cody-Waite reduction x = k*ln2 + r (|r| <= ln2/2, ln2 split
// into a head with 11 trailing zero bits and a tail) and the degree-7 Taylor
// polynomial of e^r evaluated by Horner's rule, then scaled by 2^k through the
// exponent field.  Only +, -, *, rint and integer bit operations are used, so the
// host restatement of this function returns the same bits.  Max error ~1 ulp.
__host__ __device__ inline float det_expf(float x) {
  if (x > 88.72283f) return __builtin_huge_valf();
  if (x < -103.97208f) return 0.0f;
  const float kf = rintf(x * 1.44269504088896341f);
  const float ln2_hi = 0.693145751953125f;          // 0x3F317200
  const float ln2_lo = 1.42860682030941723212e-6f;  // ln2 - ln2_hi
  const float r = (x - kf * ln2_hi) - kf * ln2_lo;
  float p = 1.0f / 5040.0f;
  p = p * r + 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  int k = (int)kf;
  if (k > 127) {  // only reachable just below the overflow threshold
    p = p * 2.0f;
    k -= 1;
  }
  if (k < -126) {  // gradual underflow: scale in two exact steps
    p = p * 1.17549435e-38f;  // 2^-126
    k += 126;
  }
  union {
    uint32_t u;
    float f;
  } s;
  s.u = (uint32_t)(k + 127) << 23;
  return p * s.f;
}

// jax.nn.sigmoid restated as 1 / (1 + exp(-x)).
__host__ __device__ inline float det_sigmoidf(float x) { return 1.0f / (1.0f + det_expf(-x)); }

__host__ __device__ inline float bits_to_float(uint32_t u) {
  union {
    uint32_t u;
    float f;
  } v;
  v.u = u;
  return v.f;
}
__host__ __device__ inline uint32_t float_to_bits(float f) {
  union {
    uint32_t u;
    float f;
  } v;
  v.f = f;
  return v.u;
}

// jnp.minimum / jnp.maximum / jnp.clip propagate NaN.
__device__ inline float jmax(float a, float b) { return (a != a || b != b) ? (a + b) : (a > b ? a : b); }
__device__ inline float jmin(float a, float b) { return (a != a || b != b) ? (a + b) : (a < b ? a : b); }

// Cotangent share of the first operand of jnp.maximum(a, b) / jnp.minimum(a, b):
// JAX autodiff splits the cotangent equally at a tie.
__device__ inline float dmax_first(float a, float b) { return a > b ? 1.0f : (a == b ? 0.5f : 0.0f); }
__device__ inline float dmin_first(float a, float b) { return a < b ? 1.0f : (a == b ? 0.5f : 0.0f); }

// Real spherical-harmonic constants of degrees 0..3 (sh.py:6-22), the standard
// orthonormal basis normalisations sqrt((2l+1)/(4pi) * (l-|m|)!/(l+|m|)!) with the
// sign convention of the 3DGS colour model.
constexpr float SH_C0 = 0.28209479177387814f;
constexpr float SH_C1 = 0.4886025119029199f;
constexpr float SH_C2_0 = 1.0925484305920792f;
constexpr float SH_C2_1 = -1.0925484305920792f;
constexpr float SH_C2_2 = 0.31539156525252005f;
constexpr float SH_C2_3 = -1.0925484305920792f;
constexpr float SH_C2_4 = 0.5462742152960396f;
constexpr float SH_C3_0 = -0.5900435899266435f;
constexpr float SH_C3_1 = 2.890611442640554f;
constexpr float SH_C3_2 = -0.4570457994644658f;
constexpr float SH_C3_3 = 0.3731763325901154f;
constexpr float SH_C3_4 = -0.4570457994644658f;
constexpr float SH_C3_5 = 1.445305721320277f;
constexpr float SH_C3_6 = -0.5900435899266435f;

inline int div_up(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

}  // namespace gs

// ---- error reporting shared by the C entry points -------------------------------
namespace gs {
void set_error(const char* fmt, ...);
int hip_check(hipError_t e, const char* what);
int launch_check(const char* what);
}  // namespace gs

#define GS_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      gs::set_error(__VA_ARGS__);      \
      return GS_ERR_INVALID;           \
    }                                  \
  } while (0)

#define GS_LAUNCH_CHECK(name)                   \
  do {                                          \
    int _rc = gs::launch_check(name);           \
    if (_rc != GS_OK) return _rc;               \
  } while (0)
