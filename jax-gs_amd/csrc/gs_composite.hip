// Per-tile alpha compositing on gfx950 (forward and backward).
//
// Reference: jax_gs/renderer/rasterizer.py:157-248 (render_tiles): a pixel centre is
// (16*tx + i + 0.5, 16*ty + j + 0.5); the first min(count, 4096) entries of a tile
// are blended front to back; entry k is blended iff T > 1e-4 before it and its
// power > -10, with alpha = min(0.99, exp(power) * sigmoid(opacity)); the pixel is
// C + T * background.  rasterizer_tpu.py computes the same image.
//
// Work decomposition: every wave owns PPT*4 rows of one 16x16 tile; lane l holds the
// PPT pixels (l % 16, row0 + l / 16 + 4 i), i < PPT, i.e. one column, so the x offset
// to a Gaussian is shared by the lane's pixels.  Waves are independent (no LDS, no
// barriers).  The entry a wave works on is the same for all its lanes, so its id and
// its 48-byte record come in through scalar loads straight into SGPRs (prefetched one
// and two entries ahead) and feed the vector math as scalar operands.  With PPT = 4 a
// wave covers the whole tile (used for large images); PPT = 1 uses four waves per
// tile for small images that would otherwise leave CUs idle.
//
// Forward: branch-free per pixel (an entry blends iff T > 1e-4 before it and its
// power > -10); the wave stops when every pixel has T <= 1e-4 (ballot every 8
// entries).  Per pixel it writes the final T and n_contrib, the number of leading
// entries met while T > 1e-4.
// Backward: replays each pixel back to front from (final T, n_contrib), recovering
// T_k = T_{k+1} / (1 - alpha_k) and the colour behind entry k,
// R_{k-1} = alpha_k c_k + (1 - alpha_k) R_k.  The 9 gradient terms of an entry are
// summed over the lane's pixels, reduce-scattered across the wave (recursive halving,
// so lane c ends with the total of term c) and added to the Gaussian's gradient
// record with one atomic instruction (9 lanes).  Gradients follow JAX autodiff of the
// reference: the cap
// min(0.99, .) passes no gradient when it binds (half at a tie), gated entries pass
// none.
#include "gs_common.h"

namespace gs {
namespace {

constexpr float kTMin = 1e-4f;
constexpr float kLog2e = 1.4426950408889634f;

__device__ inline float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ inline float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ inline int bcast_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

__device__ inline float dpp_add(float x, int t) { return x + __int_as_float(t); }

// Sum over the 64 lanes; the total is returned in every lane (through an SGPR).
// Row reduction with row_shr 1,2,4,8 leaves each 16-lane row's sum in its lane 15;
// row_bcast:15 and row_bcast:31 fold the rows into lane 63.
__device__ inline float wave_sum(float v) {
  float x = v;
  x = dpp_add(x, __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xF, 0xF, false));
  x = dpp_add(x, __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xF, 0xF, false));
  x = dpp_add(x, __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xF, 0xF, false));
  x = dpp_add(x, __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xF, 0xF, false));
  x = dpp_add(x, __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xA, 0xF, false));
  x = dpp_add(x, __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xC, 0xF, false));
  return bcast(x, 63);
}

// Reduce-scatter of 9 per-lane values over the wave by recursive halving: at level
// k a lane keeps the half of its values whose index bit k equals its own lane bit k
// and adds the partner's copy of them (partner = lane ^ 2^k: DPP quad_perm for
// 1 and 2, ds_swizzle for 4, 8, 16, ds_bpermute for 32).  Afterwards lane L holds
// the wave total of value L % 16 (values 9..15 are zero padding).
__device__ inline float swz_xor(float v, int pattern_xor) {
  // ds_swizzle bit mode: and_mask 0x1F, or_mask 0, xor_mask in bits 14:10
  switch (pattern_xor) {
    case 4: return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (4 << 10) | 0x1F));
    case 8: return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (8 << 10) | 0x1F));
    default: return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (16 << 10) | 0x1F));
  }
}

__device__ inline float reduce_scatter9(const float* v, int lane) {
  const bool b0 = lane & 1, b1 = lane & 2, b2 = lane & 4, b3 = lane & 8;
  float y[5], z[3], r[2];
  // level 0: xor 1 (quad_perm [1,0,3,2])
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    const float lo = v[2 * k];
    const float hi = (2 * k + 1 < 9) ? v[2 * k + 1] : 0.0f;
    const float keep = b0 ? hi : lo, send = b0 ? lo : hi;
    y[k] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0xB1, 0xF, 0xF, false));
  }
  // level 1: xor 2 (quad_perm [2,3,0,1])
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    const float lo = y[2 * m];
    const float hi = (2 * m + 1 < 5) ? y[2 * m + 1] : 0.0f;
    const float keep = b1 ? hi : lo, send = b1 ? lo : hi;
    z[m] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x4E, 0xF, 0xF, false));
  }
  // level 2: xor 4
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float lo = z[2 * q];
    const float hi = (2 * q + 1 < 3) ? z[2 * q + 1] : 0.0f;
    const float keep = b2 ? hi : lo, send = b2 ? lo : hi;
    r[q] = keep + swz_xor(send, 4);
  }
  // level 3: xor 8
  float t;
  {
    const float keep = b3 ? r[1] : r[0], send = b3 ? r[0] : r[1];
    t = keep + swz_xor(send, 8);
  }
  // levels 4, 5: full sums across the 16-lane rows
  t = t + swz_xor(t, 16);
  t = t + __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __float_as_int(t)));
  return t;
}

// XCD-aware tile order: consecutive workgroups go round-robin to the 8 XCDs, so
// workgroup b works on tile (b % 8) * per + b / 8 and each XCD's L2 sees a contiguous
// band of tiles that share Gaussians.
__device__ inline int tile_of_block(int b, int T) {
  const int per = (T + 7) >> 3;
  return (b & 7) * per + (b >> 3);
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

struct Rec {
  float mx, my, A, B, C, op, r, g, b;
};

__device__ inline Rec zero_rec() { return Rec{0, 0, 0, 0, 0, 0, 0, 0, 0}; }

__device__ inline Rec load_rec(const float4* __restrict__ rec, int g) {
  const float4 a = rec[(int64_t)g * 3];
  const float4 b = rec[(int64_t)g * 3 + 1];
  const float c = rec[(int64_t)g * 3 + 2].x;
  return Rec{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c};
}

// power = -0.5 * (ic00 dx^2 + 2 ic01 dx dy + ic11 dy^2) with the -0.5 folded into the
// record (A, B, C); the forward and backward kernels share this exact expression.
__device__ inline float power_of(float dy, float Adx2, float Bdx, float C) {
  return fmaf(C * dy, dy, fmaf(Bdx, dy, Adx2));
}

// Gaussian id of entry k of the tile (uniform: scalar load).  Ids are clamped like
// XLA's gather only where they are used, so that the load is not waited for early.
__device__ inline int entry_gid(const int32_t* __restrict__ gids, int start, int k) { return gids[start + k]; }
__device__ inline int clamp_gid(int g, int num_g) { return min(max(g, 0), num_g - 1); }

template <int PPT>
__global__ __launch_bounds__(64) void composite_fwd_kernel(
    const float4* __restrict__ rec, int num_g, const int32_t* __restrict__ gids, int64_t n_entries,
    const int32_t* __restrict__ ranges, int W, int H, int TX, int T, const float* __restrict__ bg,
    float* __restrict__ img, float* __restrict__ finalT, int32_t* __restrict__ ncontrib) {
  constexpr int WPT = 4 / PPT;  // waves per tile
  const int b = blockIdx.x / WPT, part = blockIdx.x % WPT;
  const int tile = tile_of_block(b, T);
  if (tile >= T) return;
  const int lane = threadIdx.x;
  const int tx = tile % TX, ty = tile / TX;
  const int X = tx * kTile + (lane & 15);
  const int Y0 = ty * kTile + part * 4 * PPT + (lane >> 4);
  const float px = (float)(tx * kTile) + ((float)(lane & 15) + 0.5f);
  float py[PPT], Tr[PPT], c0[PPT], c1[PPT], c2[PPT];
  int cnt[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int yl = part * 4 * PPT + (lane >> 4) + 4 * i;
    py[i] = (float)(ty * kTile) + ((float)yl + 0.5f);
    // pixels outside the image start "finished" so they never hold the wave
    Tr[i] = (X < W && Y0 + 4 * i < H) ? 1.0f : 0.0f;
    c0[i] = c1[i] = c2[i] = 0.0f;
    cnt[i] = 0;
  }
  int start, n;
  tile_span(ranges, tile, n_entries, num_g, start, n);

  // Entry k's id and record are wave-uniform: scalar loads, the record fetched one
  // entry ahead and the id two entries ahead so neither load stalls the wave.
  Rec nxt = zero_rec();
  int gnext = 0;
  if (n > 0) nxt = load_rec(rec, clamp_gid(entry_gid(gids, start, 0), num_g));
  if (n > 1) gnext = entry_gid(gids, start, 1);
  for (int k = 0; k < n; ++k) {
    const Rec e = nxt;
    if (k + 1 < n) nxt = load_rec(rec, clamp_gid(gnext, num_g));
    if (k + 2 < n) gnext = entry_gid(gids, start, k + 2);
    const float dx = px - e.mx;
    const float Adx2 = (e.A * dx) * dx, Bdx = e.B * dx;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const float dy = py[i] - e.my;
      const float pw = power_of(dy, Adx2, Bdx, e.C);
      const bool act = Tr[i] > kTMin;  // rasterizer.py:206
      float al = fast_exp(pw) * e.op;
      al = al < 0.99f ? al : 0.99f;
      al = (act && pw > -10.0f) ? al : 0.0f;  // rasterizer.py:212
      const float w = al * Tr[i];
      c0[i] = fmaf(w, e.r, c0[i]);
      c1[i] = fmaf(w, e.g, c1[i]);
      c2[i] = fmaf(w, e.b, c2[i]);
      Tr[i] = Tr[i] * (1.0f - al);
      cnt[i] += act ? 1 : 0;
    }
    if ((k & 7) == 7) {
      bool live = false;
#pragma unroll
      for (int i = 0; i < PPT; ++i) live = live || Tr[i] > kTMin;
      if (__ballot(live) == 0ull) break;
    }
  }
  const float bg0 = bg[0], bg1 = bg[1], bg2 = bg[2];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int Y = Y0 + 4 * i;
    if (X < W && Y < H) {
      const int64_t p = (int64_t)Y * W + X;
      img[3 * p] = c0[i] + Tr[i] * bg0;
      img[3 * p + 1] = c1[i] + Tr[i] * bg1;
      img[3 * p + 2] = c2[i] + Tr[i] * bg2;
      if (finalT) finalT[p] = Tr[i];
      if (ncontrib) ncontrib[p] = cnt[i];
    }
  }
}

template <int PPT>
__global__ __launch_bounds__(64) void composite_bwd_kernel(
    const float4* __restrict__ rec, int num_g, const int32_t* __restrict__ gids, int64_t n_entries,
    const int32_t* __restrict__ ranges, int W, int H, int TX, int T, const float* __restrict__ bg,
    const float* __restrict__ gimg, const float* __restrict__ finalT, const int32_t* __restrict__ ncontrib,
    float* __restrict__ grec, float* __restrict__ gbg) {
  constexpr int WPT = 4 / PPT;
  const int b = blockIdx.x / WPT, part = blockIdx.x % WPT;
  const int tile = tile_of_block(b, T);
  if (tile >= T) return;
  const int lane = threadIdx.x;
  const int tx = tile % TX, ty = tile / TX;
  const int X = tx * kTile + (lane & 15);
  const int Y0 = ty * kTile + part * 4 * PPT + (lane >> 4);
  const float px = (float)(tx * kTile) + ((float)(lane & 15) + 0.5f);
  int start, n;
  tile_span(ranges, tile, n_entries, num_g, start, n);
  const float bg0 = bg[0], bg1 = bg[1], bg2 = bg[2];

  float py[PPT], Tr[PPT], g0[PPT], g1[PPT], g2[PPT], R0[PPT], R1[PPT], R2[PPT];
  int kp[PPT];
  int kmax = 0;
  float tb0 = 0.0f, tb1 = 0.0f, tb2 = 0.0f;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int yl = part * 4 * PPT + (lane >> 4) + 4 * i;
    py[i] = (float)(ty * kTile) + ((float)yl + 0.5f);
    Tr[i] = 1.0f;
    g0[i] = g1[i] = g2[i] = 0.0f;
    kp[i] = 0;
    const int Y = Y0 + 4 * i;
    if (X < W && Y < H) {
      const int64_t p = (int64_t)Y * W + X;
      Tr[i] = finalT[p];
      const int k = ncontrib[p];
      kp[i] = k < 0 ? 0 : (k > n ? n : k);  // entries beyond the tile's list never load
      g0[i] = gimg[3 * p];
      g1[i] = gimg[3 * p + 1];
      g2[i] = gimg[3 * p + 2];
    }
    R0[i] = bg0;
    R1[i] = bg1;
    R2[i] = bg2;
    kmax = max(kmax, kp[i]);
    // dL/dbackground = sum over pixels of T_final * g
    tb0 = fmaf(Tr[i], g0[i], tb0);
    tb1 = fmaf(Tr[i], g1[i], tb1);
    tb2 = fmaf(Tr[i], g2[i], tb2);
  }
  if (gbg != nullptr) {
    const float s0 = wave_sum(tb0), s1 = wave_sum(tb1), s2 = wave_sum(tb2);
    if (lane < 3) atomicAdd(&gbg[lane], lane == 0 ? s0 : (lane == 1 ? s1 : s2));
  }
  // wave-wide maximum entry count (uniform loop bound)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) kmax = max(kmax, __shfl_xor(kmax, o, 64));
  kmax = bcast_i(kmax, 0);

  // entries kmax-1 .. 0, ids and records by scalar loads (uniform), prefetched
  Rec nxt = zero_rec();
  int gcur = 0, gnext = 0;
  if (kmax > 0) {
    gcur = clamp_gid(entry_gid(gids, start, kmax - 1), num_g);
    nxt = load_rec(rec, gcur);
  }
  if (kmax > 1) gnext = entry_gid(gids, start, kmax - 2);
  for (int k = kmax - 1; k >= 0; --k) {
    const Rec e = nxt;
    const int g = gcur;
    if (k >= 1) {
      gcur = clamp_gid(gnext, num_g);
      nxt = load_rec(rec, gcur);
    }
    if (k >= 2) gnext = entry_gid(gids, start, k - 2);
    const float dx = px - e.mx;
    const float Adx2 = (e.A * dx) * dx, Bdx = e.B * dx;
    float v[9];
#pragma unroll
    for (int c = 0; c < 9; ++c) v[c] = 0.0f;
    bool any = false;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const float dy = py[i] - e.my;
      const float pw = power_of(dy, Adx2, Bdx, e.C);
      if (k < kp[i] && pw > -10.0f) {
        any = true;
        const float ex = fast_exp(pw);
        const float araw = ex * e.op;
        const float al = araw < 0.99f ? araw : 0.99f;
        const float capf = araw < 0.99f ? 1.0f : (araw == 0.99f ? 0.5f : 0.0f);
        const float om = 1.0f - al;
        const float Tk = Tr[i] * __builtin_amdgcn_rcpf(om);
        const float w = al * Tk;
        v[6] = fmaf(w, g0[i], v[6]);
        v[7] = fmaf(w, g1[i], v[7]);
        v[8] = fmaf(w, g2[i], v[8]);
        const float dal = Tk * fmaf(e.b - R2[i], g2[i], fmaf(e.g - R1[i], g1[i], (e.r - R0[i]) * g0[i]));
        R0[i] = fmaf(al, e.r, om * R0[i]);
        R1[i] = fmaf(al, e.g, om * R1[i]);
        R2[i] = fmaf(al, e.b, om * R2[i]);
        Tr[i] = Tk;
        const float dae = dal * capf;
        const float dpw = dae * araw;
        v[5] = fmaf(dae, ex, v[5]);
        const float dpx = dpw * dx, dpy = dpw * dy;
        v[2] = fmaf(dpx, dx, v[2]);
        v[3] = fmaf(dpx, dy, v[3]);
        v[4] = fmaf(dpy, dy, v[4]);
        // d power / d mean = -(2 A dx + B dy, B dx + 2 C dy)
        v[0] = fmaf(-dpw, fmaf(2.0f * e.A, dx, e.B * dy), v[0]);
        v[1] = fmaf(-dpw, fmaf(e.B, dx, 2.0f * e.C * dy), v[1]);
      }
    }
    if (__ballot(any) != 0ull) {
      const float mine = reduce_scatter9(v, lane);
      if (lane < 9 && mine != 0.0f) atomicAdd(&grec[(int64_t)g * kRec + lane], mine);
    }
  }
}

__global__ void zero_f32_kernel(float* __restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.0f;
}

// Large images have enough tiles to fill the GPU with one wave per tile.
inline int pick_ppt(int T) { return T >= 2048 ? 4 : 1; }

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gs_composite_fwd(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                                int64_t n_entries, const int32_t* ranges, int width, int height,
                                const float* background, float* image, float* final_T, int32_t* n_contrib) {
  GS_REQUIRE(n >= 0 && n < ((int64_t)1 << 31), "gs_composite_fwd: n out of range");
  GS_REQUIRE(n_entries >= 0, "gs_composite_fwd: n_entries must be >= 0");
  GS_REQUIRE(width > 0 && height > 0, "gs_composite_fwd: bad image size %dx%d", width, height);
  GS_REQUIRE(ranges && background && image, "gs_composite_fwd: NULL argument");
  GS_REQUIRE(n == 0 || n_entries == 0 || (records && sorted_gids), "gs_composite_fwd: NULL records/gids");
  const int TX = (width + kTile - 1) / kTile, TY = (height + kTile - 1) / kTile;
  const int T = TX * TY;
  const int nblk = ((T + 7) / 8) * 8;
  hipStream_t s = (hipStream_t)stream;
  if (pick_ppt(T) == 4) {
    hipLaunchKernelGGL(composite_fwd_kernel<4>, dim3(nblk), dim3(64), 0, s, (const float4*)records, (int)n,
                       sorted_gids, n_entries, ranges, width, height, TX, T, background, image, final_T, n_contrib);
  } else {
    hipLaunchKernelGGL(composite_fwd_kernel<1>, dim3(nblk * 4), dim3(64), 0, s, (const float4*)records, (int)n,
                       sorted_gids, n_entries, ranges, width, height, TX, T, background, image, final_T, n_contrib);
  }
  GS_LAUNCH_CHECK("composite_fwd_kernel");
  return GS_OK;
}

extern "C" int gs_composite_bwd(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                                int64_t n_entries, const int32_t* ranges, int width, int height,
                                const float* background, const float* grad_image, const float* final_T,
                                const int32_t* n_contrib, float* grad_records, float* grad_background) {
  GS_REQUIRE(n >= 0 && n < ((int64_t)1 << 31), "gs_composite_bwd: n out of range");
  GS_REQUIRE(n_entries >= 0, "gs_composite_bwd: n_entries must be >= 0");
  GS_REQUIRE(width > 0 && height > 0, "gs_composite_bwd: bad image size %dx%d", width, height);
  GS_REQUIRE(ranges && background && grad_image && final_T && n_contrib, "gs_composite_bwd: NULL argument");
  GS_REQUIRE(n == 0 || n_entries == 0 || (records && sorted_gids && grad_records),
             "gs_composite_bwd: NULL records/gids");
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
  if (pick_ppt(T) == 4) {
    hipLaunchKernelGGL(composite_bwd_kernel<4>, dim3(nblk), dim3(64), 0, s, (const float4*)records, (int)n,
                       sorted_gids, n_entries, ranges, width, height, TX, T, background, grad_image, final_T,
                       n_contrib, grad_records, grad_background);
  } else {
    hipLaunchKernelGGL(composite_bwd_kernel<1>, dim3(nblk * 4), dim3(64), 0, s, (const float4*)records, (int)n,
                       sorted_gids, n_entries, ranges, width, height, TX, T, background, grad_image, final_T,
                       n_contrib, grad_records, grad_background);
  }
  GS_LAUNCH_CHECK("composite_bwd_kernel");
  return GS_OK;
}
