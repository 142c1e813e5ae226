// Tile binning on gfx950: the integer half of the rasterizer.
//
// Reference: jax_gs/renderer/rasterizer.py:12-116 (get_tile_interactions) and
// jax_gs/renderer/renderer.py:57-90 (tile ranges + health extras).  The reference
// materialises 256 slots per Gaussian, packs key = (tile << 13) | (bits(depth) >> 18)
// and runs one stable sort over all 256*N slots.  Its output order is therefore
// (tile, depth bucket, Gaussian id).  This file produces the same order for the
// valid entries with far less data movement:
//
//   1. bin_prep         per Gaussian: tile rectangle (clipped to 16x16 tiles), entry
//                        count and 13-bit depth bucket; radius-cap / sign stats.
//   2. depth sort       stable counting sort of the N Gaussians by depth bucket
//                        (two 8-bit LSD passes) -> Gaussians in (bucket, id) order.
//   3. count scan       exclusive scan of entry counts in that order -> offsets, M.
//   4. duplicate        each Gaussian writes its (tile, id) entries at its offset, so
//                        the entry list is in (bucket, id) order.
//   5. tile sort        stable LSD radix passes on the tile id (8-bit digits) ->
//                        (tile, bucket, id) order, exactly the reference's.
//   6. ranges + stats   searchsorted-left boundaries and the renderer's extras.
//
// The radix passes use one wave per workgroup and a fixed grid of G workgroups that
// each own a contiguous key range, so stability only needs an in-wave rank: lanes
// with equal digits are found with 8 ballots ("match any") and ranked by lane order.
#include "gs_common.h"

namespace gs {
namespace {

constexpr int kRadixBits = 8;
constexpr int kRadixBins = 1 << kRadixBits;
constexpr int kScanBlock = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanBlock * kScanItems;  // 4096 elements per scan block
constexpr int kMaxScanPartials = 1024 * 64;         // single-block scan of partials

__device__ inline uint64_t lanemask_lt() {
  const unsigned lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// ---------------------------------------------------------------------------------
// 1. per-Gaussian rectangle, count, depth bucket (rasterizer.py:36-51, 84-94;
//    renderer.py:63-75 for the radius-cap statistic).
__global__ __launch_bounds__(256) void bin_prep_kernel(int64_t n, const float* __restrict__ means2d,
                                                       const float* __restrict__ radii,
                                                       const uint8_t* __restrict__ valid,
                                                       const float* __restrict__ depths, int W, int H,
                                                       int TX, uint32_t* __restrict__ dkey,
                                                       uint2* __restrict__ rect,
                                                       int32_t* __restrict__ stats) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  bool cap_violation = false, negative = false;
  if (i < n) {
    const float mx = means2d[2 * i], my = means2d[2 * i + 1], r = radii[i];
    const float wm1 = (float)(W - 1), hm1 = (float)(H - 1);
    const float minx = jmin(jmax(mx - r, 0.0f), wm1);
    const float maxx = jmin(jmax(mx + r, 0.0f), wm1);
    const float miny = jmin(jmax(my - r, 0.0f), hm1);
    const float maxy = jmin(jmax(my + r, 0.0f), hm1);
    // floor(x/16) on values in [0, W-1] (NaN only for Gaussians that are invalid).
    const int tminx = (int)floorf(minx / 16.0f), tmaxx = (int)floorf(maxx / 16.0f);
    const int tminy = (int)floorf(miny / 16.0f), tmaxy = (int)floorf(maxy / 16.0f);
    const bool on_screen = (mx + r > 0.0f) && (mx - r < (float)W) && (my + r > 0.0f) && (my - r < (float)H);
    const bool proj_valid = valid[i] != 0;
    const bool v = proj_valid && on_screen && (tmaxx >= tminx) && (tmaxy >= tminy);
    const int spanx = tmaxx - tminx + 1, spany = tmaxy - tminy + 1;
    cap_violation = proj_valid && on_screen && (spanx > kOffset || spany > kOffset);
    const uint32_t zb = float_to_bits(depths[i]);
    negative = (zb >> 31) != 0;
    uint32_t key = kDepthBinEmpty;
    uint2 rc = make_uint2(0u, 0u);
    if (v) {
      const int w = spanx < kOffset ? spanx : kOffset;
      const int h = spany < kOffset ? spany : kOffset;
      // v implies depth > 0.01, so the 13-bit bucket is in [3848, 8191].
      key = (zb >> (31 - kDepthBits)) - kDepthBucketLo;
      rc.x = (uint32_t)tminx | ((uint32_t)tminy << 16);
      rc.y = (uint32_t)w | ((uint32_t)h << 8);
    }
    dkey[i] = key;
    rect[i] = rc;
  }
  const uint64_t capm = __ballot(cap_violation);
  const uint64_t negm = __ballot(negative);
  if ((threadIdx.x & 63) == 0) {
    if (capm) atomicAdd(&stats[GS_STAT_RADIUS_CAP_VIOLATIONS], (int)__popcll(capm));
    if (negm) atomicAdd(&stats[GS_STAT_NEGATIVE_DEPTH], (int)__popcll(negm));
  }
  (void)TX;
}

// ---------------------------------------------------------------------------------
// Device-wide exclusive scan of uint32 (3 phases, no inter-block waiting).
struct LoadPlain {
  const uint32_t* p;
  __device__ uint32_t operator()(int64_t i) const { return p[i]; }
};
// Entry count of the Gaussian at depth-sorted position i.
struct LoadSortedCount {
  const uint32_t* order;
  const uint2* rect;
  int64_t n;
  __device__ uint32_t operator()(int64_t i) const {
    const uint32_t g = order[i];
    if ((int64_t)g >= n) return 0u;  // unreachable for a permutation; keeps reads in bounds
    const uint2 rc = rect[g];
    return (rc.y & 0xFFu) * ((rc.y >> 8) & 0xFFu);
  }
};

__device__ inline uint32_t wave_incl_scan(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// Exclusive scan of one value per thread over a 256-thread block; returns the block
// total through *total.
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t* total) {
  __shared__ uint32_t wsum[4];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint32_t inc = wave_incl_scan(v);
  if (lane == 63) wsum[wid] = inc;
  __syncthreads();
  uint32_t wbase = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (k < wid) wbase += wsum[k];
    tot += wsum[k];
  }
  __syncthreads();
  *total = tot;
  return wbase + inc - v;
}

template <class Load>
__global__ __launch_bounds__(kScanBlock) void scan_reduce_kernel(Load load, int64_t n,
                                                                 uint32_t* __restrict__ partial) {
  const int64_t base = (int64_t)blockIdx.x * kScanTile + threadIdx.x;
  uint32_t s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + (int64_t)k * kScanBlock;
    if (i < n) s += load(i);
  }
  uint32_t tot;
  block_excl_scan(s, &tot);
  if (threadIdx.x == 0) partial[blockIdx.x] = tot;
}

// Single block: exclusive scan of nb partials in place; grand total to *total.
__global__ __launch_bounds__(kScanBlock) void scan_partials_kernel(uint32_t* __restrict__ partial, int nb,
                                                                   uint32_t* __restrict__ total) {
  __shared__ uint32_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int b0 = 0; b0 < nb; b0 += kScanBlock) {
    const int i = b0 + threadIdx.x;
    const uint32_t v = i < nb ? partial[i] : 0u;
    uint32_t tot;
    const uint32_t ex = block_excl_scan(v, &tot);
    const uint32_t c = carry;
    if (i < nb) partial[i] = c + ex;
    __syncthreads();
    if (threadIdx.x == 0) carry = c + tot;
    __syncthreads();
  }
  if (threadIdx.x == 0 && total != nullptr) *total = carry;
}

// Blocked layout: thread t owns elements [t*16, t*16+16) of the block's tile so the
// sequential per-thread sums compose into an exclusive scan in element order.
template <class Load>
__global__ __launch_bounds__(kScanBlock) void scan_down_kernel(Load load, int64_t n,
                                                               const uint32_t* __restrict__ partial,
                                                               uint32_t* __restrict__ out) {
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  uint32_t v[kScanItems];
  uint32_t s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    v[k] = i < n ? load(i) : 0u;
    s += v[k];
  }
  uint32_t tot;
  uint32_t run = partial[blockIdx.x] + block_excl_scan(s, &tot);
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    if (i < n) out[i] = run;
    run += v[k];
  }
}

// ---------------------------------------------------------------------------------
// Stable LSD radix pass, 8-bit digit at `shift`.  Grid = G single-wave workgroups;
// workgroup g owns keys [g*chunk, min(n,(g+1)*chunk)).  n is min(*n_dev, cap) when
// n_dev is given (device-resident entry count), else n_static.
__device__ inline void pass_range(const uint32_t* n_dev, int64_t n_static, int64_t cap, int G,
                                  int64_t& begin, int64_t& end, int64_t* n_out = nullptr) {
  int64_t n = n_static;
  if (n_dev != nullptr) {
    n = (int64_t)(*n_dev);
    if (n > cap) n = cap;
  }
  int64_t chunk = (n + G - 1) / G;
  chunk = (chunk + 63) & ~(int64_t)63;
  begin = (int64_t)blockIdx.x * chunk;
  end = begin + chunk;
  if (end > n) end = n;
  if (n_out) *n_out = n;
}

__global__ __launch_bounds__(64) void radix_upsweep_kernel(const uint32_t* __restrict__ keys,
                                                           const uint32_t* __restrict__ n_dev,
                                                           int64_t n_static, int64_t cap, int shift,
                                                           int G, uint32_t* __restrict__ table) {
  __shared__ uint32_t hist[kRadixBins];
  const int lane = threadIdx.x;
  for (int d = lane; d < kRadixBins; d += 64) hist[d] = 0;
  __syncthreads();
  int64_t begin, end;
  pass_range(n_dev, n_static, cap, G, begin, end);
  for (int64_t i = begin + lane; i < end; i += 64) atomicAdd(&hist[(keys[i] >> shift) & (kRadixBins - 1)], 1u);
  __syncthreads();
  for (int d = lane; d < kRadixBins; d += 64) table[(int64_t)d * G + blockIdx.x] = hist[d];
}

constexpr int kUnroll = 4;

__global__ __launch_bounds__(64) void radix_downsweep_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
    const uint32_t* __restrict__ n_dev, int64_t n_static, int64_t cap, int shift, int G,
    const uint32_t* __restrict__ table, uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t cnt[kRadixBins];
  const int lane = threadIdx.x;
  for (int d = lane; d < kRadixBins; d += 64) cnt[d] = table[(int64_t)d * G + blockIdx.x];
  __syncthreads();
  int64_t begin, end, n_pass;
  pass_range(n_dev, n_static, cap, G, begin, end, &n_pass);
  const uint64_t lt = lanemask_lt();
  for (int64_t base = begin; base < end; base += 64 * kUnroll) {
    uint32_t k[kUnroll], v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * 64 + lane;
      const bool a = i < end;
      k[u] = a ? keys_in[i] : 0u;
      v[u] = a ? (vals_in ? vals_in[i] : (uint32_t)i) : 0u;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * 64 + lane;
      const bool a = i < end;
      const uint32_t d = (k[u] >> shift) & (kRadixBins - 1);
      uint64_t m = __ballot(a);
#pragma unroll
      for (int b = 0; b < kRadixBits; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bb = __ballot(bit);
        m &= bit ? bb : ~bb;
      }
      uint32_t dst = 0;
      if (a) {
        const uint64_t before = m & lt;
        const uint32_t base_d = cnt[d];
        dst = base_d + (uint32_t)__popcll(before);
        // All lanes have read cnt[] before the group's first lane writes it back:
        // LDS operations of one wave execute in program order.
        if (before == 0) cnt[d] = base_d + (uint32_t)__popcll(m);
      }
      if (a && dst < (uint32_t)n_pass) {  // always true for a consistent table
        if (keys_out) keys_out[dst] = k[u];
        vals_out[dst] = v[u];
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// 4. duplicate: Gaussian at depth-sorted position p writes its entries at off[p].
//    Slot order inside a Gaussian is row-major over its clipped rectangle
//    (rasterizer.py:56-69); each Gaussian meets a tile at most once, so this order
//    never decides a tie.
__global__ __launch_bounds__(256) void duplicate_kernel(int64_t n, const uint32_t* __restrict__ order,
                                                        const uint2* __restrict__ rect,
                                                        const uint32_t* __restrict__ off,
                                                        const uint32_t* __restrict__ n_entries, int64_t cap,
                                                        int TX, uint32_t* __restrict__ ekey,
                                                        uint32_t* __restrict__ eval) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const uint32_t g = order[p];
  if ((int64_t)g >= n) return;
  const uint2 rc = rect[g];
  const int w = rc.y & 0xFF, h = (rc.y >> 8) & 0xFF;
  const int cnt = w * h;
  if (cnt == 0) return;
  const int tminx = rc.x & 0xFFFF, tminy = rc.x >> 16;
  const int64_t o = off[p];
  (void)n_entries;
  int j = 0;
  for (int oy = 0; oy < h; ++oy) {
    const uint32_t row = (uint32_t)((tminy + oy) * TX + tminx);
    for (int ox = 0; ox < w; ++ox, ++j) {
      const int64_t e = o + j;
      if (e < cap) {
        ekey[e] = row + ox;
        eval[e] = g;
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// 6. ranges[t] = first entry with tile >= t (searchsorted-left), ranges[T] = M.
// Fixed grid, grid-stride over the device-resident entry count.
__global__ __launch_bounds__(256) void ranges_kernel(const uint32_t* __restrict__ tiles,
                                                     const uint32_t* __restrict__ n_entries, int64_t cap,
                                                     int T, int32_t* __restrict__ ranges) {
  int64_t M = *n_entries;
  if (M > cap) M = cap;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i <= M; i += stride) {
    int64_t tp = i > 0 ? (int64_t)tiles[i - 1] : -1;
    int64_t tc = i < M ? (int64_t)tiles[i] : (int64_t)T;
    if (tp < -1) tp = -1;
    if (tc > T) tc = T;
    for (int64_t t = tp + 1; t <= tc; ++t) ranges[t] = (int32_t)i;
  }
}

// Same boundary rule on a caller-provided sorted array that may hold -1 (negative
// depth) and T (sentinel) entries.
__global__ __launch_bounds__(256) void ranges_any_kernel(const int32_t* __restrict__ tiles, int64_t L, int T,
                                                         int32_t* __restrict__ ranges) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i <= L; i += stride) {
    int64_t tp = i > 0 ? (int64_t)tiles[i - 1] : -1;
    int64_t tc = i < L ? (int64_t)tiles[i] : (int64_t)T;
    if (tp < -1) tp = -1;
    if (tc > T) tc = T;
    for (int64_t t = tp + 1; t <= tc; ++t) ranges[t] = (int32_t)i;
  }
}

__global__ __launch_bounds__(256) void tile_stats_kernel(const int32_t* __restrict__ ranges, int T,
                                                         const uint32_t* __restrict__ n_entries, int64_t cap,
                                                         int32_t* __restrict__ stats) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  int cntv = 0;
  if (t < T) cntv = ranges[t + 1] - ranges[t];
  // block reductions of max / counts / sums
  __shared__ int smax[4], sot[4], soi[4], stt[4], sti[4];
  int mx = cntv;
  int ot = cntv > kBlock ? 1 : 0, oi = cntv > kBlock ? cntv - kBlock : 0;
  int tt = cntv > kMaxTileEntries ? 1 : 0, ti = cntv > kMaxTileEntries ? cntv - kMaxTileEntries : 0;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mx = max(mx, __shfl_xor(mx, o, 64));
    ot += __shfl_xor(ot, o, 64);
    oi += __shfl_xor(oi, o, 64);
    tt += __shfl_xor(tt, o, 64);
    ti += __shfl_xor(ti, o, 64);
  }
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    smax[wid] = mx; sot[wid] = ot; soi[wid] = oi; stt[wid] = tt; sti[wid] = ti;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k) {
      mx = max(smax[0], smax[k]); smax[0] = mx;
      sot[0] += sot[k]; soi[0] += soi[k]; stt[0] += stt[k]; sti[0] += sti[k];
    }
    atomicMax(&stats[GS_STAT_MAX_PER_TILE], smax[0]);
    atomicAdd(&stats[GS_STAT_OVERFLOW_TILES], sot[0]);
    atomicAdd(&stats[GS_STAT_OVERFLOW_INTERACTIONS], soi[0]);
    atomicAdd(&stats[GS_STAT_TRUNCATED_TILES], stt[0]);
    atomicAdd(&stats[GS_STAT_TRUNCATED_INTERACTIONS], sti[0]);
    if (blockIdx.x == 0) {
      const uint32_t m = *n_entries;
      stats[GS_STAT_N_INTERACTIONS] = (int32_t)m;
      stats[GS_STAT_CAPACITY_EXCEEDED] = ((int64_t)m > cap) ? 1 : 0;
    }
  }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------------
struct BinPlan {
  int64_t n, cap;
  int T, TX, TY;
  int G_n, G_m;  // radix grids for the N-sort and the M-sort
  int tile_passes;
  int nb_n;      // scan blocks over N
  int nb_table;  // scan blocks over the larger radix table
  // byte offsets into the workspace
  size_t o_dkey, o_rect, o_ka, o_va, o_kb, o_vb, o_off, o_part, o_table, o_nent, o_ek0, o_ev0, o_ek1,
      o_ev1, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

BinPlan make_plan(int64_t n, int width, int height, int64_t capacity) {
  BinPlan P;
  P.n = n;
  P.cap = capacity > 0 ? capacity : 256 * (n > 2 ? n : 2);
  P.TX = (width + kTile - 1) / kTile;
  P.TY = (height + kTile - 1) / kTile;
  P.T = P.TX * P.TY;
  int bits = 1;
  while ((1 << bits) < P.T) ++bits;
  P.tile_passes = (bits + kRadixBits - 1) / kRadixBits;
  P.G_n = (int)std::min<int64_t>(1024, std::max<int64_t>(1, (n + 4095) / 4096));
  P.G_m = 2048;
  P.nb_n = div_up(std::max<int64_t>(n, 1), kScanTile);
  const int64_t tbl = (int64_t)kRadixBins * std::max(P.G_n, P.G_m);
  P.nb_table = div_up(tbl, kScanTile);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  const size_t nn = (size_t)std::max<int64_t>(n, 1);
  P.o_dkey = take(nn * 4);
  P.o_rect = take(nn * 8);
  P.o_ka = take(nn * 4);
  P.o_va = take(nn * 4);
  P.o_kb = take(nn * 4);
  P.o_vb = take(nn * 4);
  P.o_off = take((nn + 1) * 4);
  P.o_part = take((size_t)std::max(P.nb_n, P.nb_table) * 4 + 64);
  P.o_table = take((size_t)tbl * 4);
  P.o_nent = take(64);
  P.o_ek0 = take((size_t)P.cap * 4);
  P.o_ev0 = take((size_t)P.cap * 4);
  P.o_ek1 = take((size_t)P.cap * 4);
  P.o_ev1 = take((size_t)P.cap * 4);
  P.total = o;
  return P;
}

template <class Load>
int run_scan(hipStream_t s, Load load, int64_t n, uint32_t* partial, uint32_t* out, uint32_t* total) {
  const int nb = div_up(std::max<int64_t>(n, 1), kScanTile);
  if (nb > kMaxScanPartials) {
    set_error("gs_bin: scan of %lld elements exceeds the supported size", (long long)n);
    return GS_ERR_INVALID;
  }
  hipLaunchKernelGGL(scan_reduce_kernel<Load>, dim3(nb), dim3(kScanBlock), 0, s, load, n, partial);
  GS_LAUNCH_CHECK("scan_reduce_kernel");
  hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(kScanBlock), 0, s, partial, nb, total);
  GS_LAUNCH_CHECK("scan_partials_kernel");
  hipLaunchKernelGGL(scan_down_kernel<Load>, dim3(nb), dim3(kScanBlock), 0, s, load, n, partial, out);
  GS_LAUNCH_CHECK("scan_down_kernel");
  return GS_OK;
}

// One stable radix pass: keys_in/vals_in -> keys_out/vals_out on digit `shift`.
int radix_pass(hipStream_t s, const uint32_t* kin, const uint32_t* vin, uint32_t* kout, uint32_t* vout,
               const uint32_t* n_dev, int64_t n_static, int64_t cap, int shift, int G, uint32_t* table,
               uint32_t* partial) {
  hipLaunchKernelGGL(radix_upsweep_kernel, dim3(G), dim3(64), 0, s, kin, n_dev, n_static, cap, shift, G, table);
  GS_LAUNCH_CHECK("radix_upsweep_kernel");
  int rc = run_scan(s, LoadPlain{table}, (int64_t)kRadixBins * G, partial, table, (uint32_t*)nullptr);
  if (rc != GS_OK) return rc;
  hipLaunchKernelGGL(radix_downsweep_kernel, dim3(G), dim3(64), 0, s, kin, vin, n_dev, n_static, cap, shift, G,
                     table, kout, vout);
  GS_LAUNCH_CHECK("radix_downsweep_kernel");
  return GS_OK;
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" size_t gs_bin_workspace_size(int64_t n, int width, int height, int64_t capacity) {
  if (n < 0 || width <= 0 || height <= 0) return 0;
  return make_plan(n, width, height, capacity).total;
}

extern "C" int gs_bin(void* stream, int64_t n, const float* means2d, const float* radii, const uint8_t* valid,
                      const float* depths, int width, int height, int64_t capacity, void* workspace,
                      size_t workspace_bytes, int32_t* sorted_gids, int32_t* sorted_tiles, int32_t* ranges,
                      int32_t* stats) {
  GS_REQUIRE(n >= 0 && n < (int64_t)1 << 31, "gs_bin: n must be in [0, 2^31) (got %lld)", (long long)n);
  GS_REQUIRE(width > 0 && height > 0 && width <= 65535 * kTile && height <= 65535 * kTile,
             "gs_bin: bad image size %dx%d", width, height);
  const BinPlan P = make_plan(n, width, height, capacity);
  GS_REQUIRE(P.cap < ((int64_t)1 << 31), "gs_bin: capacity %lld too large", (long long)P.cap);
  GS_REQUIRE(P.tile_passes <= 2, "gs_bin: %d tiles exceed the 65536-tile limit", P.T);
  GS_REQUIRE(workspace != nullptr && workspace_bytes >= P.total,
             "gs_bin: workspace of %zu bytes is smaller than the %zu required", workspace_bytes, P.total);
  GS_REQUIRE(sorted_gids && ranges && stats, "gs_bin: NULL output");
  GS_REQUIRE(n == 0 || (means2d && radii && valid && depths), "gs_bin: NULL input");
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  uint32_t* dkey = (uint32_t*)(ws + P.o_dkey);
  uint2* rect = (uint2*)(ws + P.o_rect);
  uint32_t* ka = (uint32_t*)(ws + P.o_ka);
  uint32_t* va = (uint32_t*)(ws + P.o_va);
  uint32_t* kb = (uint32_t*)(ws + P.o_kb);
  uint32_t* vb = (uint32_t*)(ws + P.o_vb);
  uint32_t* off = (uint32_t*)(ws + P.o_off);
  uint32_t* part = (uint32_t*)(ws + P.o_part);
  uint32_t* table = (uint32_t*)(ws + P.o_table);
  uint32_t* nent = (uint32_t*)(ws + P.o_nent);
  uint32_t* ek0 = (uint32_t*)(ws + P.o_ek0);
  uint32_t* ev0 = (uint32_t*)(ws + P.o_ev0);
  uint32_t* ek1 = (uint32_t*)(ws + P.o_ek1);
  uint32_t* ev1 = (uint32_t*)(ws + P.o_ev1);

  hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, s, stats, (int64_t)GS_NUM_STATS, 0);
  GS_LAUNCH_CHECK("fill_i32_kernel");
  if (n == 0) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(div_up(P.T + 1, 256)), dim3(256), 0, s, ranges, (int64_t)P.T + 1, 0);
    GS_LAUNCH_CHECK("fill_i32_kernel");
    return GS_OK;
  }
  // 1. prep
  hipLaunchKernelGGL(bin_prep_kernel, dim3(div_up(n, 256)), dim3(256), 0, s, n, means2d, radii, valid, depths, width,
                     height, P.TX, dkey, rect, stats);
  GS_LAUNCH_CHECK("bin_prep_kernel");
  // 2. stable depth sort of Gaussian ids: pass 1 (low byte) dkey,id -> kb,vb; pass 2 -> ka,va
  int rc = radix_pass(s, dkey, nullptr, kb, vb, nullptr, n, n, 0, P.G_n, table, part);
  if (rc != GS_OK) return rc;
  rc = radix_pass(s, kb, vb, ka, va, nullptr, n, n, 8, P.G_n, table, part);
  if (rc != GS_OK) return rc;
  const uint32_t* order = va;
  // 3. entry offsets in depth order; total -> nent
  rc = run_scan(s, LoadSortedCount{order, rect, n}, n, part, off, nent);
  if (rc != GS_OK) return rc;
  // 4. duplicate (tile, id) in depth order
  hipLaunchKernelGGL(duplicate_kernel, dim3(div_up(n, 256)), dim3(256), 0, s, n, order, rect, off, nent, P.cap,
                     P.TX, ek0, ev0);
  GS_LAUNCH_CHECK("duplicate_kernel");
  // 5. stable radix sort on the tile id
  uint32_t* tiles_out = sorted_tiles ? (uint32_t*)sorted_tiles : ek1;
  if (P.tile_passes == 1) {
    rc = radix_pass(s, ek0, ev0, tiles_out, (uint32_t*)sorted_gids, nent, 0, P.cap, 0, P.G_m, table, part);
    if (rc != GS_OK) return rc;
  } else {
    rc = radix_pass(s, ek0, ev0, ek1, ev1, nent, 0, P.cap, 0, P.G_m, table, part);
    if (rc != GS_OK) return rc;
    uint32_t* tout = sorted_tiles ? (uint32_t*)sorted_tiles : ek0;
    rc = radix_pass(s, ek1, ev1, tout, (uint32_t*)sorted_gids, nent, 0, P.cap, 8, P.G_m, table, part);
    if (rc != GS_OK) return rc;
    tiles_out = tout;
  }
  // 6. ranges + stats
  hipLaunchKernelGGL(ranges_kernel, dim3(2048), dim3(256), 0, s, tiles_out, nent, P.cap, P.T, ranges);
  GS_LAUNCH_CHECK("ranges_kernel");
  hipLaunchKernelGGL(tile_stats_kernel, dim3(div_up(P.T, 256)), dim3(256), 0, s, ranges, P.T, nent, P.cap, stats);
  GS_LAUNCH_CHECK("tile_stats_kernel");
  return GS_OK;
}

extern "C" int gs_tile_ranges(void* stream, const int32_t* sorted_tiles, int64_t length, int num_tiles,
                              int32_t* ranges) {
  GS_REQUIRE(length >= 0 && num_tiles >= 0, "gs_tile_ranges: bad sizes");
  GS_REQUIRE(ranges != nullptr && (length == 0 || sorted_tiles != nullptr), "gs_tile_ranges: NULL argument");
  hipLaunchKernelGGL(ranges_any_kernel, dim3(std::min<int64_t>(2048, div_up(length + 1, 256))), dim3(256), 0,
                     (hipStream_t)stream, sorted_tiles, length, num_tiles, ranges);
  GS_LAUNCH_CHECK("ranges_any_kernel");
  return GS_OK;
}
