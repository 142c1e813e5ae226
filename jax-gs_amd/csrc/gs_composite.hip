// Per-tile alpha compositing on gfx950 (forward and backward).
//
// Reference: jax_gs/renderer/rasterizer.py:157-248 (render_tiles): a pixel centre is
// (16*tx + i + 0.5, 16*ty + j + 0.5); the first min(count, 4096) entries of a tile
// are blended front to back; entry k is blended iff T > 1e-4 before it and its
// power > -10, with alpha = min(0.99, exp(power) * sigmoid(opacity)); the pixel is
// C + T * background.  rasterizer_tpu.py computes the same image.
//
// Layout: one 256-thread workgroup (4 waves) per 16x16 tile, one pixel per thread.
// Entries are staged through LDS in batches of 256 records (48 B each); the tile
// stops as soon as every pixel has T <= 1e-4 (workgroup-wide vote).  The backward
// replays each pixel back to front from its saved final T and entry count,
// recovering T_k = T_{k+1} / (1 - alpha_k), reduces each entry's 9 gradient terms
// across the wave, combines the 4 waves in LDS and issues one set of float atomics
// per (tile, entry).
#include "gs_common.h"

namespace gs {
namespace {

constexpr int kThreads = 256;
constexpr float kTMin = 1e-4f;

__device__ inline float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// power of rasterizer.py:210 with the -0.5 folded into the record (exact: a power
// of two scaling), same association as the reference.
__device__ inline float power_of(float dx, float dy, float4 a, float b_x) {
  return ((dx * dx) * a.z + (dx * dy) * a.w) + (dy * dy) * b_x;
}

// XCD-aware tile order: consecutive workgroups go round-robin to the 8 XCDs, so
// block b is given tile (b % 8) * per + b / 8 and each XCD's L2 sees a contiguous
// band of tiles that share Gaussians.
__device__ inline int tile_of_block(int b, int T) {
  const int per = (T + 7) >> 3;
  const int xcd = b & 7, k = b >> 3;
  const int t = xcd * per + k;
  return t;
}

// Entries [start, start+n) of a tile, n capped at 4096; ranges are clamped to the
// entry array so that inconsistent inputs cannot index outside it.
__device__ inline void tile_span(const int32_t* __restrict__ ranges, int tile, int64_t n_entries, int num_g,
                                 int& start, int& n) {
  int64_t s = ranges[tile], e = ranges[tile + 1];
  s = s < 0 ? 0 : (s > n_entries ? n_entries : s);
  e = e < s ? s : (e > n_entries ? n_entries : e);
  int64_t c = e - s;
  c = c < kMaxTileEntries ? c : kMaxTileEntries;
  start = (int)s;
  n = num_g > 0 ? (int)c : 0;
}

__global__ __launch_bounds__(kThreads) void composite_fwd_kernel(
    const float4* __restrict__ rec, int num_g, const int32_t* __restrict__ gids, int64_t n_entries,
    const int32_t* __restrict__ ranges, int W, int H, int TX, int T, const float* __restrict__ bg,
    float* __restrict__ img,
    float* __restrict__ finalT, int32_t* __restrict__ ncontrib) {
  const int tile = tile_of_block(blockIdx.x, T);
  if (tile >= T) return;  // uniform per workgroup
  const int tx = tile % TX, ty = tile / TX;
  const int lx = threadIdx.x & 15, ly = threadIdx.x >> 4;
  const int pix = tx * kTile + lx, piy = ty * kTile + ly;
  const bool inside = pix < W && piy < H;
  const float px = (float)(tx * kTile) + ((float)lx + 0.5f);
  const float py = (float)(ty * kTile) + ((float)ly + 0.5f);
  int start, n;
  tile_span(ranges, tile, n_entries, num_g, start, n);

  __shared__ float4 sA[kThreads], sB[kThreads];
  __shared__ float sC[kThreads];
  float T_ = 1.0f, c0 = 0.0f, c1 = 0.0f, c2 = 0.0f;
  int kstop = 0;
  bool done = !inside;
  for (int b0 = 0; b0 < n; b0 += kThreads) {
    if (__syncthreads_count(done) == kThreads) break;
    const int k = b0 + threadIdx.x;
    if (k < n) {
      // out-of-range ids clamp, as XLA's gather does
      const int g = min(max(gids[start + k], 0), num_g - 1);
      const float4* r = rec + (int64_t)g * 3;
      sA[threadIdx.x] = r[0];
      sB[threadIdx.x] = r[1];
      sC[threadIdx.x] = r[2].x;
    }
    __syncthreads();
    if (!done) {
      const int cnt = (n - b0) < kThreads ? (n - b0) : kThreads;
      int j = 0;
      for (; j < cnt; ++j) {
        const float4 a = sA[j];
        const float4 b = sB[j];
        const float dx = px - a.x, dy = py - a.y;
        const float pw = power_of(dx, dy, a, b.x);
        if (pw > -10.0f) {
          float al = fast_exp(pw) * b.y;
          al = al < 0.99f ? al : 0.99f;
          const float wgt = al * T_;
          c0 = c0 + wgt * b.z;
          c1 = c1 + wgt * b.w;
          c2 = c2 + wgt * sC[j];
          T_ = T_ * (1.0f - al);
          if (T_ <= kTMin) {
            done = true;
            ++j;
            break;
          }
        }
      }
      kstop = b0 + j;
    }
  }
  if (inside) {
    const int64_t p = (int64_t)piy * W + pix;
    img[3 * p] = c0 + T_ * bg[0];
    img[3 * p + 1] = c1 + T_ * bg[1];
    img[3 * p + 2] = c2 + T_ * bg[2];
    if (finalT) finalT[p] = T_;
    if (ncontrib) ncontrib[p] = kstop;
  }
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__global__ __launch_bounds__(kThreads) void composite_bwd_kernel(
    const float4* __restrict__ rec, int num_g, const int32_t* __restrict__ gids, int64_t n_entries,
    const int32_t* __restrict__ ranges, int W, int H, int TX, int T, const float* __restrict__ bg,
    const float* __restrict__ gimg,
    const float* __restrict__ finalT, const int32_t* __restrict__ ncontrib, float* __restrict__ grec,
    float* __restrict__ gbg) {
  const int tile = tile_of_block(blockIdx.x, T);
  if (tile >= T) return;
  const int tx = tile % TX, ty = tile / TX;
  const int lx = threadIdx.x & 15, ly = threadIdx.x >> 4;
  const int pix = tx * kTile + lx, piy = ty * kTile + ly;
  const bool inside = pix < W && piy < H;
  const float px = (float)(tx * kTile) + ((float)lx + 0.5f);
  const float py = (float)(ty * kTile) + ((float)ly + 0.5f);
  int start, n;
  tile_span(ranges, tile, n_entries, num_g, start, n);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;

  float T_ = 1.0f, g0 = 0.0f, g1 = 0.0f, g2 = 0.0f;
  int kp = 0;
  if (inside) {
    const int64_t p = (int64_t)piy * W + pix;
    T_ = finalT[p];
    kp = ncontrib[p];
    kp = kp < 0 ? 0 : (kp > n ? n : kp);  // entries beyond the tile's list never load
    g0 = gimg[3 * p];
    g1 = gimg[3 * p + 1];
    g2 = gimg[3 * p + 2];
  }
  const float bg0 = bg[0], bg1 = bg[1], bg2 = bg[2];
  // dL/dbackground = sum_p T_final(p) * g(p)
  if (gbg != nullptr) {
    float t0 = wave_sum(T_ * g0), t1 = wave_sum(T_ * g1), t2 = wave_sum(T_ * g2);
    if (lane == 0) {
      atomicAdd(&gbg[0], t0);
      atomicAdd(&gbg[1], t1);
      atomicAdd(&gbg[2], t2);
    }
  }
  float R0 = bg0, R1 = bg1, R2 = bg2;  // colour behind the current entry, per unit T

  __shared__ int skmax[4];
  int km = kp;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) km = max(km, __shfl_xor(km, o, 64));
  if (lane == 0) skmax[wid] = km;
  __syncthreads();
  const int kmax = max(max(skmax[0], skmax[1]), max(skmax[2], skmax[3]));

  __shared__ float4 sA[kThreads], sB[kThreads];
  __shared__ float sC[kThreads];
  __shared__ int sG[kThreads];
  __shared__ float sgrad[9][kThreads];
  for (int b1 = kmax; b1 > 0; b1 -= kThreads) {
    const int b0 = b1 > kThreads ? b1 - kThreads : 0;
    const int cnt = b1 - b0;
    if ((int)threadIdx.x < cnt) {
      const int g = min(max(gids[start + b0 + threadIdx.x], 0), num_g - 1);
      const float4* r = rec + (int64_t)g * 3;
      sG[threadIdx.x] = g;
      sA[threadIdx.x] = r[0];
      sB[threadIdx.x] = r[1];
      sC[threadIdx.x] = r[2].x;
    }
#pragma unroll
    for (int c = 0; c < 9; ++c) sgrad[c][threadIdx.x] = 0.0f;
    __syncthreads();
    for (int j = cnt - 1; j >= 0; --j) {
      const int k = b0 + j;
      float v[9];
#pragma unroll
      for (int c = 0; c < 9; ++c) v[c] = 0.0f;
      bool contrib = false;
      if (k < kp) {
        const float4 a = sA[j];
        const float4 b = sB[j];
        const float cb = sC[j];
        const float dx = px - a.x, dy = py - a.y;
        const float pw = power_of(dx, dy, a, b.x);
        if (pw > -10.0f) {
          contrib = true;
          const float e = fast_exp(pw);
          const float araw = e * b.y;
          const float al = araw < 0.99f ? araw : 0.99f;
          const float capf = araw < 0.99f ? 1.0f : (araw == 0.99f ? 0.5f : 0.0f);
          const float om = 1.0f - al;
          const float Tk = T_ / om;
          const float wgt = al * Tk;
          v[6] = wgt * g0;
          v[7] = wgt * g1;
          v[8] = wgt * g2;
          const float dal = Tk * (((b.z - R0) * g0 + (b.w - R1) * g1) + (cb - R2) * g2);
          R0 = al * b.z + om * R0;
          R1 = al * b.w + om * R1;
          R2 = al * cb + om * R2;
          T_ = Tk;
          const float dpw = dal * araw * capf;
          v[5] = dal * e * capf;
          v[2] = dpw * dx * dx;
          v[3] = dpw * dx * dy;
          v[4] = dpw * dy * dy;
          v[0] = -dpw * (2.0f * a.z * dx + a.w * dy);
          v[1] = -dpw * (a.w * dx + 2.0f * b.x * dy);
        }
      }
      if (__ballot(contrib) != 0ull) {
#pragma unroll
        for (int c = 0; c < 9; ++c) v[c] = wave_sum(v[c]);
        if (lane == 0) {
#pragma unroll
          for (int c = 0; c < 9; ++c) atomicAdd(&sgrad[c][j], v[c]);
        }
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < 9 * cnt; idx += kThreads) {
      const int j = idx / 9, c = idx - 9 * j;
      const float val = sgrad[c][j];
      if (val != 0.0f) atomicAdd(&grec[(int64_t)sG[j] * kRec + c], val);
    }
    __syncthreads();
  }
}

__global__ void zero_f32_kernel(float* __restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.0f;
}

__global__ void fill_bg_kernel(const float* __restrict__ bg, float* __restrict__ img, int64_t npix) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < npix; i += stride) {
    img[3 * i] = bg[0];
    img[3 * i + 1] = bg[1];
    img[3 * i + 2] = bg[2];
  }
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gs_composite_fwd(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                                int64_t n_entries, const int32_t* ranges, int width, int height, const float* background,
                                float* image, float* final_T, int32_t* n_contrib) {
  GS_REQUIRE(n >= 0, "gs_composite_fwd: n must be >= 0");
  GS_REQUIRE(width > 0 && height > 0, "gs_composite_fwd: bad image size %dx%d", width, height);
  GS_REQUIRE(ranges && background && image, "gs_composite_fwd: NULL argument");
  GS_REQUIRE(n == 0 || (records && sorted_gids), "gs_composite_fwd: NULL records/gids");
  const int TX = (width + kTile - 1) / kTile, TY = (height + kTile - 1) / kTile;
  const int T = TX * TY;
  const int nblk = ((T + 7) / 8) * 8;
  hipLaunchKernelGGL(composite_fwd_kernel, dim3(nblk), dim3(kThreads), 0, (hipStream_t)stream,
                     (const float4*)records, (int)n, sorted_gids, n_entries, ranges, width, height, TX, T,
                     background, image, final_T, n_contrib);
  GS_LAUNCH_CHECK("composite_fwd_kernel");
  return GS_OK;
}

extern "C" int gs_composite_bwd(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                                int64_t n_entries, const int32_t* ranges, int width, int height, const float* background,
                                const float* grad_image, const float* final_T, const int32_t* n_contrib,
                                float* grad_records, float* grad_background) {
  GS_REQUIRE(n >= 0, "gs_composite_bwd: n must be >= 0");
  GS_REQUIRE(width > 0 && height > 0, "gs_composite_bwd: bad image size %dx%d", width, height);
  GS_REQUIRE(ranges && background && grad_image && final_T && n_contrib, "gs_composite_bwd: NULL argument");
  GS_REQUIRE(n == 0 || (records && sorted_gids && grad_records), "gs_composite_bwd: NULL records/gids");
  hipStream_t s = (hipStream_t)stream;
  if (n > 0) {
    hipLaunchKernelGGL(zero_f32_kernel, dim3(1024), dim3(256), 0, s, grad_records, n * kRec);
    GS_LAUNCH_CHECK("zero_f32_kernel");
  }
  if (grad_background) {
    hipLaunchKernelGGL(zero_f32_kernel, dim3(1), dim3(64), 0, s, grad_background, (int64_t)3);
    GS_LAUNCH_CHECK("zero_f32_kernel");
  }
  const int TX = (width + kTile - 1) / kTile, TY = (height + kTile - 1) / kTile;
  const int T = TX * TY;
  const int nblk = ((T + 7) / 8) * 8;
  hipLaunchKernelGGL(composite_bwd_kernel, dim3(nblk), dim3(kThreads), 0, s, (const float4*)records, (int)n,
                     sorted_gids, n_entries, ranges, width, height, TX, T, background, grad_image, final_T, n_contrib, grad_records,
                     grad_background);
  GS_LAUNCH_CHECK("composite_bwd_kernel");
  return GS_OK;
}
