// L1 and SSIM photometric losses of a rendered image, and their gradient, on gfx950.
//
// Reference: jax_gs/training/losses.py:4-8 (l1_loss) and :16-75 (ssim, d_ssim_loss),
// combined by jax_gs/training/trainer.py:18-26 as (1 - 0.2) l1 + 0.2 d_ssim.
//   taps    w_k = exp(-k^2 / 4.5) / sum, k = -5..5 (window 11, sigma 1.5)
//   blur    correlation with w along H, then along W, 'SAME' zero padding
//   mu1 = blur(x), mu2 = blur(y), s11 = max(0, blur(x^2) - mu1^2),
//   s22 = max(0, blur(y^2) - mu2^2), s12 = blur(x y) - mu1 mu2
//   map = (2 mu1 mu2 + C1)(2 s12 + C2) / ((mu1^2 + mu2^2 + C1)(s11 + s22 + C2)),
//   C1 = 0.01^2, C2 = 0.03^2, clipped to [-1, 1]; ssim = mean over H x W x C.
//
// Forward (one launch + a final sum): a workgroup owns 16 x 54 outputs of every channel.
// The vertical pass runs over 64 columns (54 + 2 x 5 halo): each thread takes one
// column and 4 output rows, reads the 14 input rows it needs once and keeps the five
// blurred products (x, y, x^2, y^2, x y) in registers; they meet in LDS, where the
// horizontal pass (each thread 4 adjacent outputs of one row, 128-bit LDS reads of
// its 14-column window) completes the blur.  Per output the map, |x - y| and, when a
// gradient is wanted, the map's derivatives with respect to (mu1, blur(x^2),
// blur(x y)) -- divided by the count and gated by the clip -- are formed; the
// derivatives go to three planes of the workspace.
// Backward: dL/dx = blur(d/dmu1) + 2 x blur(d/dblur(x^2)) + y blur(d/dblur(x y)) (the
// blur is a correlation with a symmetric kernel and zero padding, so it is its own
// adjoint), scaled by the cotangent of the mean SSIM, plus the L1 cotangent times
// sign(x - y) / count.  Same tiling over the three planes.
// Ties follow JAX: max(0, .) and the clip pass half the cotangent at equality.
#include "gs_common.h"

namespace gs {
namespace {

constexpr int kSR = 5;                   // window radius
constexpr int kSTaps = 2 * kSR + 1;      // 11 taps
constexpr int kSTH = 16;                 // output rows per workgroup
constexpr int kSCols = 64;               // columns of the vertical pass
constexpr int kSTW = kSCols - 2 * kSR;   // 54 output columns per workgroup
constexpr int kSPad = kSCols + 4;        // LDS row (the last window reads 2 columns past 64)
constexpr float kC1 = 0.01f * 0.01f;
constexpr float kC2 = 0.03f * 0.03f;

struct Taps {
  float w[kSTaps];
};

__device__ inline float tie_step(float z) { return z > 0.0f ? 1.0f : (z == 0.0f ? 0.5f : 0.0f); }

// Vertical pass of NM maps for image column col: acc[m][o] = sum_k w_k v_m(row0 + o + k),
// o < 4, where v_m(r) = load(m, r) inside the image and 0 outside.
template <int NM, typename Load>
__device__ inline void vertical4(const Taps& t, int row0, int H, bool col_in, Load load, float (&acc)[NM][4]) {
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int o = 0; o < 4; ++o) acc[m][o] = 0.0f;
#pragma unroll
  for (int i = 0; i < 4 + 2 * kSR; ++i) {
    const int r = row0 + i;
    float v[NM];
    load(col_in && r >= 0 && r < H, r, v);
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      const int k = i - o;
      if (k >= 0 && k < kSTaps) {
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[m][o] = fmaf(t.w[k], v[m], acc[m][o]);
      }
    }
  }
}

// Horizontal pass from LDS row `row` of NM maps: out[m][o] = sum_k w_k V[m][row][c0 + o + k].
template <int NM>
__device__ inline void horizontal4(const Taps& t, const float (*V)[kSTH][kSPad], int row, int c0, float (&out)[NM][4]) {
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    float win[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 f = *reinterpret_cast<const float4*>(&V[m][row][c0 + 4 * q]);
      win[4 * q] = f.x;
      win[4 * q + 1] = f.y;
      win[4 * q + 2] = f.z;
      win[4 * q + 3] = f.w;
    }
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      float a = 0.0f;
#pragma unroll
      for (int k = 0; k < kSTaps; ++k) a = fmaf(t.w[k], win[o + k], a);
      out[m][o] = a;
    }
    __asm__ volatile("" ::: "memory");  // one map's window in registers at a time
  }
}

__device__ inline float block_sum256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// XCD-aware tile order: consecutive workgroups go round-robin to the 8 XCDs; workgroup
// b takes tile (b % 8) * per + b / 8, so each XCD's L2 holds a band of tile rows and
// the halo rows two vertically adjacent tiles share are fetched once.
__device__ inline int ssim_tile_of_block(int b, int T) { return (b & 7) * ((T + 7) >> 3) + (b >> 3); }

// Forward, CC channels (1..4), one channel at a time (the next channel's loads hit the
// cache).  The gradient maps of a channel are staged in LDS and leave as whole rows.
template <int CC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void l1_ssim_fwd_kernel(
    int H, int W, int TX, int T, const float* __restrict__ x, const float* __restrict__ y, Taps taps,
    float inv_count, float* __restrict__ gmap, float2* __restrict__ partial) {
  __shared__ __align__(16) float V[5][kSTH][kSPad];
  __shared__ float Gs[3][kSTH][kSTW];
  __shared__ float red[4];
  const int tile = ssim_tile_of_block(blockIdx.x, T);
  if (tile >= T) return;
  const int tid = threadIdx.x;
  const int ox = (tile % TX) * kSTW;  // first output column
  const int r0 = (tile / TX) * kSTH;  // first output row
  // columns 64..67 of every LDS row feed only outputs past the tile: keep them finite
  for (int i = tid; i < 5 * kSTH * 4; i += 256) V[i / (kSTH * 4)][(i / 4) % kSTH][kSCols + (i & 3)] = 0.0f;
  const int vj = tid & 63, vq = tid >> 6;  // vertical pass: column, group of 4 rows
  const int vcol = ox - kSR + vj;
  const bool vcol_in = vcol >= 0 && vcol < W;
  const int hr = tid >> 4, hs = tid & 15;  // horizontal pass: row, group of 4 columns
  const bool h_on = 4 * hs < kSTW;
  const int plane = H * W * CC;  // one gradient map, channel-planar [CC][H][W]
  float l1_acc = 0.0f, ss_acc = 0.0f;
#pragma unroll 1
  for (int ch = 0; ch < CC; ++ch) {
    float a[5][4];
    vertical4<5>(taps, r0 + 4 * vq - kSR, H, vcol_in,
                 [&](bool in, int r, float* v) {
                   const int o = (r * W + vcol) * CC + ch;  // 3 * count < 2^31 (checked by the host)
                   const float xv = in ? x[o] : 0.0f, yv = in ? y[o] : 0.0f;
                   v[0] = xv;
                   v[1] = yv;
                   v[2] = xv * xv;
                   v[3] = yv * yv;
                   v[4] = xv * yv;
                 },
                 a);
    if (ch > 0) __syncthreads();  // the previous channel is done with V and Gs
#pragma unroll
    for (int m = 0; m < 5; ++m)
#pragma unroll
      for (int o = 0; o < 4; ++o) V[m][4 * vq + o][vj] = a[m][o];
    __syncthreads();
    if (h_on) {
      float b[5][4];
      horizontal4<5>(taps, V, hr, 4 * hs, b);
      const int orow = r0 + hr;
#pragma unroll
      for (int o = 0; o < 4; ++o) {
        const int tc = 4 * hs + o, ocol = ox + tc;
        if (tc >= kSTW || ocol >= W || orow >= H) continue;
        const float mu1 = b[0][o], mu2 = b[1][o];
        const float m11 = mu1 * mu1, m22 = mu2 * mu2, m12 = mu1 * mu2;
        const float d11 = b[2][o] - m11;
        const float s11 = fmaxf(0.0f, d11), s22 = fmaxf(0.0f, b[3][o] - m22);
        const float s12 = b[4][o] - m12;
        const float A = 2.0f * m12 + kC1, B = 2.0f * s12 + kC2;
        const float Cc = (m11 + m22) + kC1, D = (s11 + s22) + kC2;
        const float num = A * B, den = Cc * D;
        // one reciprocal for the three quotients (den >= C1 C2 > 0; ~1 ulp)
        const float rden = __builtin_amdgcn_rcpf(den);
        const float raw = num * rden;
        ss_acc += fminf(1.0f, fmaxf(-1.0f, raw));
        const int p = (orow * W + ocol) * CC + ch;
        l1_acc += fabsf(x[p] - y[p]);
        // d map / d(mu1, blur(x^2), blur(x y)), times the clip gate and 1 / count
        const float G = inv_count * (tie_step(raw + 1.0f) * tie_step(1.0f - raw));
        const float dnum = G * rden, dden = -(G * raw) * rden;
        const float dA = dnum * B, dB = dnum * A, dCc = dden * D, dD = dden * Cc;
        const float de12 = 2.0f * dB;
        const float dm12 = 2.0f * dA - de12;
        const float de11 = dD * tie_step(d11);
        const float dm11 = dCc - de11;
        Gs[0][hr][tc] = 2.0f * mu1 * dm11 + mu2 * dm12;
        Gs[1][hr][tc] = de11;
        Gs[2][hr][tc] = de12;
      }
    }
    if (gmap != nullptr) {
      __syncthreads();
      // wave w writes rows w, w + 4, ... of the 3 x 16 staged rows, one value per lane
      const int lane = tid & 63, wv = tid >> 6;
      const int ncol = min(kSTW, W - ox);
      for (int row = wv; row < 3 * kSTH; row += 4) {
        const int m = row / kSTH, rr = row % kSTH, orow = r0 + rr;
        if (orow < H && lane < ncol) gmap[m * plane + (ch * H + orow) * W + ox + lane] = Gs[m][rr][lane];
      }
    }
  }
  const float l1s = block_sum256(l1_acc, red);
  const float sss = block_sum256(ss_acc, red);
  if (tid == 0) partial[tile] = make_float2(l1s, sss);
}

// out[0] = sum of |x - y| / count, out[1] = sum of the clipped map / count.
__global__ __launch_bounds__(1024) void l1_ssim_sum_kernel(const float2* __restrict__ partial, int nb,
                                                           float inv_count, float* __restrict__ out) {
  __shared__ float red[2][16];
  float a = 0.0f, b = 0.0f;
  for (int i = threadIdx.x; i < nb; i += 1024) {
    const float2 v = partial[i];
    a += v.x;
    b += v.y;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    a += __shfl_xor(a, o, 64);
    b += __shfl_xor(b, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = a;
    red[1][threadIdx.x >> 6] = b;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float s = 0.0f;
    for (int w = 0; w < 16; ++w) s += red[threadIdx.x][w];
    out[threadIdx.x] = s * inv_count;
  }
}

// Backward: the image gradient of the tile (every channel) is staged in LDS and leaves
// as whole rows.
template <int CC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void l1_ssim_bwd_kernel(
    int H, int W, int TX, int T, const float* __restrict__ x, const float* __restrict__ y, Taps taps,
    float inv_count, const float* __restrict__ gmap, const float* __restrict__ grad_out,
    float* __restrict__ grad) {
  __shared__ __align__(16) float V[3][kSTH][kSPad];
  __shared__ float Go[kSTH][kSTW * CC];
  const int tile = ssim_tile_of_block(blockIdx.x, T);
  if (tile >= T) return;
  const int tid = threadIdx.x;
  const int ox = (tile % TX) * kSTW, r0 = (tile / TX) * kSTH;
  for (int i = tid; i < 3 * kSTH * 4; i += 256) V[i / (kSTH * 4)][(i / 4) % kSTH][kSCols + (i & 3)] = 0.0f;
  const int vj = tid & 63, vq = tid >> 6;
  const int vcol = ox - kSR + vj;
  const bool vcol_in = vcol >= 0 && vcol < W;
  const int hr = tid >> 4, hs = tid & 15;
  const bool h_on = 4 * hs < kSTW;
  const int plane = H * W * CC;
  const float g_l1 = grad_out[0] * inv_count, g_ss = grad_out[1];
#pragma unroll 1
  for (int ch = 0; ch < CC; ++ch) {
    float a[3][4];
    vertical4<3>(taps, r0 + 4 * vq - kSR, H, vcol_in,
                 [&](bool in, int r, float* v) {
                   const int q = (ch * H + r) * W + vcol;
                   v[0] = in ? gmap[q] : 0.0f;
                   v[1] = in ? gmap[plane + q] : 0.0f;
                   v[2] = in ? gmap[2 * plane + q] : 0.0f;
                 },
                 a);
    if (ch > 0) __syncthreads();
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int o = 0; o < 4; ++o) V[m][4 * vq + o][vj] = a[m][o];
    __syncthreads();
    if (h_on) {
      float b[3][4];
      horizontal4<3>(taps, V, hr, 4 * hs, b);
      const int orow = r0 + hr;
#pragma unroll
      for (int o = 0; o < 4; ++o) {
        const int tc = 4 * hs + o, ocol = ox + tc;
        if (tc >= kSTW || ocol >= W || orow >= H) continue;
        const int p = (orow * W + ocol) * CC + ch;
        const float xv = x[p], yv = y[p], d = xv - yv;
        const float sg = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
        const float gs = b[0][o] + 2.0f * xv * b[1][o] + yv * b[2][o];
        Go[hr][tc * CC + ch] = g_ss * gs + g_l1 * sg;
      }
    }
  }
  __syncthreads();
  // wave w writes rows w, w + 4, ...: a row is min(54, W - ox) * CC contiguous values
  const int lane = tid & 63, wv = tid >> 6;
  const int wcols = min(kSTW, W - ox) * CC;
  for (int rr = wv; rr < kSTH; rr += 4) {
    const int orow = r0 + rr;
    if (orow >= H) break;
    float* __restrict__ dst = grad + (orow * W + ox) * CC;
    for (int cc = lane; cc < wcols; cc += 64) dst[cc] = Go[rr][cc];
  }
}

// trainer.py:18-26 from the two means: terms[0] = d_ssim = max(0, (1 - ssim) / 2),
// terms[1] = total = (1 - lambda) l1 + lambda d_ssim, and the cotangents of (l1, ssim)
// for a unit cotangent of the total: terms[2] = 1 - lambda, terms[3] = -lambda/2 times
// max's derivative (1 above 0, 1/2 at 0, as lax.max), and terms[4] = the reported metric
// 1 - 2 d_ssim (trainer.py:30).  Same float32 operations as the host-side formula.
__global__ void l1_ssim_terms_kernel(const float* __restrict__ l1_ssim, float lam, float one_minus_lam,
                                     float* __restrict__ terms) {
  const float l1 = l1_ssim[0], ssim = l1_ssim[1];
  const float half = (1.0f - ssim) / 2.0f;
  const float d = fmaxf(0.0f, half);
  terms[0] = d;
  terms[1] = one_minus_lam * l1 + lam * d;
  terms[2] = one_minus_lam;
  const float gate = half > 0.0f ? 1.0f : (half == 0.0f ? 0.5f : 0.0f);
  terms[3] = -(lam * 0.5f) * gate;
  terms[4] = 1.0f - d * 2.0f;
}

// ---------------------------------------------------------------------------------
// Any window size (losses.py:16 window_size; the trainer uses 11, served above).  The
// taps are w_j = exp(-(j - L/2)^2 / 4.5) / sum for j < L (x = arange(L) - L//2), and
// XLA's 'SAME' correlation pads (L - 1) / 2 before and L / 2 after, so output i reads
// input i + j - lo with lo = (L - 1) / 2 (for even L the window is not centred).  Planes
// are channel-planar [C][H][W] in the workspace: V (5 vertical blurs), then G (the 3
// gradient maps, as in the 11-tap path); one thread per value, the reads of a pass hit the
// cache.  The backward applies the adjoint correlation, in_s = sum_j w_j out_{s - j + lo},
// to G along W and then H (the two passes act on different axes and commute).
constexpr int kMaxTaps = 63;
struct TapsAny {
  float w[kMaxTaps];
  int L, lo;
};

// vertical blur of x, y, x^2, y^2, x y; x, y interleaved [H][W][C]
__global__ __launch_bounds__(256) void ssim_any_vblur_kernel(int H, int W, int C, const float* __restrict__ x,
                                                             const float* __restrict__ y, TapsAny t,
                                                             float* __restrict__ V) {
  const int64_t n = (int64_t)H * W * C;
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= n) return;
  const int col = (int)(q % W), r = (int)((q / W) % H), ch = (int)(q / ((int64_t)W * H));
  float a[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int j = 0; j < t.L; ++j) {
    const int rr = r + j - t.lo;
    if (rr < 0 || rr >= H) continue;
    const int64_t o = ((int64_t)rr * W + col) * C + ch;
    const float xv = x[o], yv = y[o];
    a[0] = fmaf(t.w[j], xv, a[0]);
    a[1] = fmaf(t.w[j], yv, a[1]);
    a[2] = fmaf(t.w[j], xv * xv, a[2]);
    a[3] = fmaf(t.w[j], yv * yv, a[3]);
    a[4] = fmaf(t.w[j], xv * yv, a[4]);
  }
#pragma unroll
  for (int m = 0; m < 5; ++m) V[m * n + q] = a[m];
}

// horizontal blur, the map, |x - y|, per-workgroup sums and (G != NULL) the gradient maps
__global__ __launch_bounds__(256) void ssim_any_map_kernel(int H, int W, int C, const float* __restrict__ x,
                                                           const float* __restrict__ y, TapsAny t,
                                                           const float* __restrict__ V, float inv_count,
                                                           float* __restrict__ G, float2* __restrict__ partial) {
  __shared__ float red[4];
  const int64_t n = (int64_t)H * W * C;
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  float l1v = 0.0f, ssv = 0.0f;
  if (q < n) {
    const int col = (int)(q % W), r = (int)((q / W) % H), ch = (int)(q / ((int64_t)W * H));
    float b[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < t.L; ++j) {
      const int cc = col + j - t.lo;
      if (cc < 0 || cc >= W) continue;
#pragma unroll
      for (int m = 0; m < 5; ++m) b[m] = fmaf(t.w[j], V[m * n + q - col + cc], b[m]);
    }
    const float mu1 = b[0], mu2 = b[1];
    const float m11 = mu1 * mu1, m22 = mu2 * mu2, m12 = mu1 * mu2;
    const float d11 = b[2] - m11;
    const float s11 = fmaxf(0.0f, d11), s22 = fmaxf(0.0f, b[3] - m22);
    const float s12 = b[4] - m12;
    const float A = 2.0f * m12 + kC1, B = 2.0f * s12 + kC2;
    const float Cc = (m11 + m22) + kC1, D = (s11 + s22) + kC2;
    const float num = A * B, den = Cc * D;
    const float raw = num / den;
    ssv = fminf(1.0f, fmaxf(-1.0f, raw));
    const int64_t p = ((int64_t)r * W + col) * C + ch;
    l1v = fabsf(x[p] - y[p]);
    if (G != nullptr) {
      const float Gc = inv_count * (tie_step(raw + 1.0f) * tie_step(1.0f - raw));
      const float dnum = Gc / den, dden = -(Gc * raw) / den;
      const float dA = dnum * B, dB = dnum * A, dCc = dden * D, dD = dden * Cc;
      const float de12 = 2.0f * dB;
      const float dm12 = 2.0f * dA - de12;
      const float de11 = dD * tie_step(d11);
      const float dm11 = dCc - de11;
      G[q] = 2.0f * mu1 * dm11 + mu2 * dm12;
      G[n + q] = de11;
      G[2 * n + q] = de12;
    }
  }
  const float l1s = block_sum256(l1v, red);
  const float sss = block_sum256(ssv, red);
  if (threadIdx.x == 0) partial[blockIdx.x] = make_float2(l1s, sss);
}

// adjoint correlation of the 3 gradient maps along W
__global__ __launch_bounds__(256) void ssim_any_hadj_kernel(int H, int W, int C, TapsAny t,
                                                            const float* __restrict__ G, float* __restrict__ U) {
  const int64_t n = (int64_t)H * W * C;
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= n) return;
  const int col = (int)(q % W);
  float a[3] = {0.0f, 0.0f, 0.0f};
  for (int j = 0; j < t.L; ++j) {
    const int cc = col - j + t.lo;
    if (cc < 0 || cc >= W) continue;
#pragma unroll
    for (int m = 0; m < 3; ++m) a[m] = fmaf(t.w[j], G[m * n + q - col + cc], a[m]);
  }
#pragma unroll
  for (int m = 0; m < 3; ++m) U[m * n + q] = a[m];
}

// adjoint along H, then dL/dx = g_ssim (B0 + 2 x B1 + y B2) + g_l1 sign(x - y) / count
__global__ __launch_bounds__(256) void ssim_any_grad_kernel(int H, int W, int C, const float* __restrict__ x,
                                                            const float* __restrict__ y, TapsAny t,
                                                            const float* __restrict__ U, float inv_count,
                                                            const float* __restrict__ grad_out,
                                                            float* __restrict__ grad) {
  const int64_t n = (int64_t)H * W * C;
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= n) return;
  const int col = (int)(q % W), r = (int)((q / W) % H), ch = (int)(q / ((int64_t)W * H));
  float b[3] = {0.0f, 0.0f, 0.0f};
  for (int j = 0; j < t.L; ++j) {
    const int rr = r - j + t.lo;
    if (rr < 0 || rr >= H) continue;
#pragma unroll
    for (int m = 0; m < 3; ++m) b[m] = fmaf(t.w[j], U[m * n + q + (int64_t)(rr - r) * W], b[m]);
  }
  const int64_t p = ((int64_t)r * W + col) * C + ch;
  const float xv = x[p], yv = y[p], d = xv - yv;
  const float sg = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
  const float gs = b[0] + 2.0f * xv * b[1] + yv * b[2];
  grad[p] = grad_out[1] * gs + (grad_out[0] * inv_count) * sg;
}

TapsAny make_taps_any(int L) {
  TapsAny t;
  double s = 0.0, e[kMaxTaps];
  for (int j = 0; j < L; ++j) {
    const double d = (double)(j - L / 2);
    e[j] = std::exp(-d * d / (2.0 * 1.5 * 1.5));
    s += e[j];
  }
  for (int j = 0; j < kMaxTaps; ++j) t.w[j] = j < L ? (float)(e[j] / s) : 0.0f;
  t.L = L;
  t.lo = (L - 1) / 2;
  return t;
}

struct AnyLayout {
  int64_t count;
  int nblk;
  size_t v_off, g_off, part_off, total;
};

AnyLayout any_layout(int H, int W, int C) {
  AnyLayout A;
  A.count = (int64_t)H * W * C;
  A.nblk = div_up(A.count, 256);
  A.v_off = 0;
  A.g_off = ((size_t)5 * A.count * sizeof(float) + 255) & ~(size_t)255;
  A.part_off = A.g_off + (((size_t)3 * A.count * sizeof(float) + 255) & ~(size_t)255);
  A.total = A.part_off + (size_t)A.nblk * sizeof(float2);
  return A;
}

Taps make_taps() {
  Taps t;
  double s = 0.0, e[kSTaps];
  for (int k = 0; k < kSTaps; ++k) {
    const double d = (double)(k - kSR);
    e[k] = std::exp(-d * d / (2.0 * 1.5 * 1.5));
    s += e[k];
  }
  for (int k = 0; k < kSTaps; ++k) t.w[k] = (float)(e[k] / s);
  return t;
}

struct SsimLayout {
  int64_t count;
  int TX, T;  // tiles per row, tiles
  dim3 grid;
  size_t gmap_off, part_off, total;
};

SsimLayout ssim_layout(int H, int W, int C) {
  SsimLayout L;
  L.count = (int64_t)H * W * C;
  L.TX = div_up(W, kSTW);
  L.T = L.TX * div_up(H, kSTH);
  L.grid = dim3((unsigned)(div_up(L.T, 8) * 8));
  L.gmap_off = 0;
  L.part_off = ((size_t)3 * L.count * sizeof(float) + 255) & ~(size_t)255;
  L.total = L.part_off + (size_t)L.T * sizeof(float2);
  return L;
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" size_t gs_l1_ssim_workspace_size(int height, int width, int channels) {
  if (height <= 0 || width <= 0 || channels <= 0 || channels > 4) return 0;
  return ssim_layout(height, width, channels).total;
}

extern "C" int gs_l1_ssim(void* stream, int height, int width, int channels, const float* pred,
                          const float* target, float* out, int with_grad, void* workspace, size_t workspace_bytes) {
  GS_REQUIRE(height > 0 && width > 0 && channels > 0 && channels <= 4, "gs_l1_ssim: bad image shape %dx%dx%d",
             height, width, channels);
  GS_REQUIRE(pred && target && out && workspace, "gs_l1_ssim: NULL argument");
  GS_REQUIRE(3 * (int64_t)height * width * channels < ((int64_t)1 << 31),
             "gs_l1_ssim: image %dx%dx%d too large", height, width, channels);
  const SsimLayout L = ssim_layout(height, width, channels);
  GS_REQUIRE(workspace_bytes >= L.total, "gs_l1_ssim: workspace of %zu bytes, %zu needed", workspace_bytes, L.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const float inv = (float)(1.0 / (double)L.count);
  float2* part = (float2*)(ws + L.part_off);
  float* gmap = with_grad ? (float*)(ws + L.gmap_off) : nullptr;
  const Taps taps = make_taps();
  switch (channels) {
    case 1: hipLaunchKernelGGL(l1_ssim_fwd_kernel<1>, L.grid, dim3(256), 0, s, height, width, L.TX, L.T, pred, target, taps, inv, gmap, part); break;
    case 2: hipLaunchKernelGGL(l1_ssim_fwd_kernel<2>, L.grid, dim3(256), 0, s, height, width, L.TX, L.T, pred, target, taps, inv, gmap, part); break;
    case 3: hipLaunchKernelGGL(l1_ssim_fwd_kernel<3>, L.grid, dim3(256), 0, s, height, width, L.TX, L.T, pred, target, taps, inv, gmap, part); break;
    default: hipLaunchKernelGGL(l1_ssim_fwd_kernel<4>, L.grid, dim3(256), 0, s, height, width, L.TX, L.T, pred, target, taps, inv, gmap, part); break;
  }
  GS_LAUNCH_CHECK("l1_ssim_fwd_kernel");
  hipLaunchKernelGGL(l1_ssim_sum_kernel, dim3(1), dim3(1024), 0, s, (const float2*)part, L.T, inv, out);
  GS_LAUNCH_CHECK("l1_ssim_sum_kernel");
  return GS_OK;
}

extern "C" int gs_l1_ssim_bwd(void* stream, int height, int width, int channels, const float* pred,
                              const float* target, const float* grad_out, const void* workspace,
                              size_t workspace_bytes, float* grad_pred) {
  GS_REQUIRE(height > 0 && width > 0 && channels > 0 && channels <= 4,
             "gs_l1_ssim_bwd: bad image shape %dx%dx%d", height, width, channels);
  GS_REQUIRE(pred && target && grad_out && workspace && grad_pred, "gs_l1_ssim_bwd: NULL argument");
  GS_REQUIRE(3 * (int64_t)height * width * channels < ((int64_t)1 << 31),
             "gs_l1_ssim_bwd: image %dx%dx%d too large", height, width, channels);
  const SsimLayout L = ssim_layout(height, width, channels);
  GS_REQUIRE(workspace_bytes >= L.total, "gs_l1_ssim_bwd: workspace of %zu bytes, %zu needed", workspace_bytes,
             L.total);
  hipStream_t s = (hipStream_t)stream;
  const float inv = (float)(1.0 / (double)L.count);
  const float* gmap = (const float*)((const char*)workspace + L.gmap_off);
  const Taps taps = make_taps();
  switch (channels) {
    case 1: hipLaunchKernelGGL(l1_ssim_bwd_kernel<1>, L.grid, dim3(256), 0, s, height, width, L.TX, L.T, pred, target, taps, inv, gmap, grad_out, grad_pred); break;
    case 2: hipLaunchKernelGGL(l1_ssim_bwd_kernel<2>, L.grid, dim3(256), 0, s, height, width, L.TX, L.T, pred, target, taps, inv, gmap, grad_out, grad_pred); break;
    case 3: hipLaunchKernelGGL(l1_ssim_bwd_kernel<3>, L.grid, dim3(256), 0, s, height, width, L.TX, L.T, pred, target, taps, inv, gmap, grad_out, grad_pred); break;
    default: hipLaunchKernelGGL(l1_ssim_bwd_kernel<4>, L.grid, dim3(256), 0, s, height, width, L.TX, L.T, pred, target, taps, inv, gmap, grad_out, grad_pred); break;
  }
  GS_LAUNCH_CHECK("l1_ssim_bwd_kernel");
  return GS_OK;
}

extern "C" int gs_l1_ssim_terms(void* stream, const float* l1_ssim, double lambda_ssim, float* terms) {
  GS_REQUIRE(l1_ssim && terms, "gs_l1_ssim_terms: NULL argument");
  GS_REQUIRE(lambda_ssim >= 0.0 && lambda_ssim <= 1.0, "gs_l1_ssim_terms: lambda must be in [0, 1]");
  hipLaunchKernelGGL(l1_ssim_terms_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, l1_ssim, (float)lambda_ssim,
                     (float)(1.0 - lambda_ssim), terms);
  GS_LAUNCH_CHECK("l1_ssim_terms_kernel");
  return GS_OK;
}

extern "C" size_t gs_l1_ssim_window_workspace_size(int height, int width, int channels, int window_size) {
  if (height <= 0 || width <= 0 || channels <= 0 || window_size < 1 || window_size > kMaxTaps) return 0;
  return any_layout(height, width, channels).total;
}

extern "C" int gs_l1_ssim_window(void* stream, int height, int width, int channels, int window_size,
                                 const float* pred, const float* target, float* out, int with_grad, void* workspace,
                                 size_t workspace_bytes) {
  GS_REQUIRE(height > 0 && width > 0 && channels > 0, "gs_l1_ssim_window: bad image shape %dx%dx%d", height, width,
             channels);
  GS_REQUIRE(window_size >= 1 && window_size <= kMaxTaps, "gs_l1_ssim_window: window_size must be in [1, %d] (got %d)",
             kMaxTaps, window_size);
  GS_REQUIRE(pred && target && out && workspace, "gs_l1_ssim_window: NULL argument");
  GS_REQUIRE(5 * (int64_t)height * width * channels < ((int64_t)1 << 40), "gs_l1_ssim_window: image too large");
  const AnyLayout A = any_layout(height, width, channels);
  GS_REQUIRE(workspace_bytes >= A.total, "gs_l1_ssim_window: workspace of %zu bytes, %zu needed", workspace_bytes,
             A.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const TapsAny t = make_taps_any(window_size);
  const float inv = (float)(1.0 / (double)A.count);
  float* V = (float*)(ws + A.v_off);
  float* G = with_grad ? (float*)(ws + A.g_off) : nullptr;
  float2* part = (float2*)(ws + A.part_off);
  hipLaunchKernelGGL(ssim_any_vblur_kernel, dim3(A.nblk), dim3(256), 0, s, height, width, channels, pred, target, t,
                     V);
  GS_LAUNCH_CHECK("ssim_any_vblur_kernel");
  hipLaunchKernelGGL(ssim_any_map_kernel, dim3(A.nblk), dim3(256), 0, s, height, width, channels, pred, target, t,
                     (const float*)V, inv, G, part);
  GS_LAUNCH_CHECK("ssim_any_map_kernel");
  hipLaunchKernelGGL(l1_ssim_sum_kernel, dim3(1), dim3(1024), 0, s, (const float2*)part, A.nblk, inv, out);
  GS_LAUNCH_CHECK("l1_ssim_sum_kernel");
  return GS_OK;
}

extern "C" int gs_l1_ssim_window_bwd(void* stream, int height, int width, int channels, int window_size,
                                     const float* pred, const float* target, const float* grad_out, void* workspace,
                                     size_t workspace_bytes, float* grad_pred) {
  GS_REQUIRE(height > 0 && width > 0 && channels > 0, "gs_l1_ssim_window_bwd: bad image shape %dx%dx%d", height,
             width, channels);
  GS_REQUIRE(window_size >= 1 && window_size <= kMaxTaps,
             "gs_l1_ssim_window_bwd: window_size must be in [1, %d] (got %d)", kMaxTaps, window_size);
  GS_REQUIRE(pred && target && grad_out && workspace && grad_pred, "gs_l1_ssim_window_bwd: NULL argument");
  const AnyLayout A = any_layout(height, width, channels);
  GS_REQUIRE(workspace_bytes >= A.total, "gs_l1_ssim_window_bwd: workspace of %zu bytes, %zu needed",
             workspace_bytes, A.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const TapsAny t = make_taps_any(window_size);
  const float inv = (float)(1.0 / (double)A.count);
  const float* G = (const float*)(ws + A.g_off);
  float* U = (float*)(ws + A.v_off);  // the forward's vertical blurs are dead by now
  hipLaunchKernelGGL(ssim_any_hadj_kernel, dim3(A.nblk), dim3(256), 0, s, height, width, channels, t, G, U);
  GS_LAUNCH_CHECK("ssim_any_hadj_kernel");
  hipLaunchKernelGGL(ssim_any_grad_kernel, dim3(A.nblk), dim3(256), 0, s, height, width, channels, pred, target, t,
                     (const float*)U, inv, grad_out, grad_pred);
  GS_LAUNCH_CHECK("ssim_any_grad_kernel");
  return GS_OK;
}
