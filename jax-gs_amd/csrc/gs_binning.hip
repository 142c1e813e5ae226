// Tile binning on gfx950: the integer half of the rasterizer.
//
// Reference: jax_gs/renderer/rasterizer.py:12-116 (get_tile_interactions) and
// jax_gs/renderer/renderer.py:57-90 (tile ranges + health extras).  The reference
// materialises 256 slots per Gaussian, packs key = (tile << 13) | (bits(depth) >> 18)
// and runs one stable sort over all 256*N slots, so its valid entries come out in
// (tile, 13-bit depth bucket, Gaussian id) order.  This file produces exactly that
// order without sorting the entries themselves:
//
//   1. bin_prep        per Gaussian: tile rectangle (clipped to 16x16 tiles) and depth
//                      bucket; per-block counts of radius-cap violations and negative
//                      depths (no same-address atomics).
//   2. depth sort      stable LSD radix sort of the N Gaussian ids by depth bucket
//                      (two 7-bit passes)            -> Gaussians in (bucket, id) order.
//   3. superblocks     every Gaussian meets at most 5x5 "superblocks" of 4x4 tiles;
//                      its (superblock, id) pairs are written in depth order and
//                      stably sorted by superblock (two 7-bit passes) -> per superblock
//                      the list of Gaussians touching it, in (bucket, id) order.
//   4. tile pass       a superblock's list is cut into chunks of 256 Gaussians; a wave
//                      takes a chunk 64 Gaussians at a time, forms 4 column and 4 row
//                      lane masks with ballots, and so knows for each of the 16 tiles
//                      which lanes hit it.  A counting sweep gives per (chunk, tile)
//                      counts, a scan over tiles gives the tile ranges and per-chunk
//                      offsets, and a writing sweep stores each entry's Gaussian id at
//                      offset + popcount(mask & lanes-below) -- stable by construction.
//   5. stats           the renderer's health extras from the ranges.
//
// Radix passes use one wave per workgroup and a fixed grid of G workgroups that each
// own a contiguous key range, so stability only needs an in-wave rank: lanes with
// equal digits are found with ballots ("match any") and ranked by lane order.
#include "gs_common.h"

#include <algorithm>

namespace gs {
namespace {

constexpr int kRadixBits = 7;
constexpr int kRadixBins = 1 << kRadixBits;
constexpr int kScanBlock = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanBlock * kScanItems;  // 4096 elements per scan block
constexpr int kMaxScanPartials = 1024 * 64;         // single-block scan of partials
constexpr int kSB = 4;                              // superblock = 4x4 tiles
constexpr int kSBMax = 5 * 5;                       // superblocks one Gaussian can meet
constexpr int kChunk = 256;                         // Gaussians per chunk of the tile pass
constexpr int kPrepBlock = 256;

__device__ inline uint64_t lanemask_lt() {
  const unsigned lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// rect.x = tminx | tminy << 16, rect.y = w | h << 8 (w, h <= 16; 0 when invalid)
__device__ inline void unpack_rect(uint2 rc, int& x0, int& y0, int& w, int& h) {
  x0 = rc.x & 0xFFFF;
  y0 = rc.x >> 16;
  w = rc.y & 0xFF;
  h = (rc.y >> 8) & 0xFF;
}

__device__ inline uint32_t sb_count(uint2 rc) {
  int x0, y0, w, h;
  unpack_rect(rc, x0, y0, w, h);
  if (w == 0 || h == 0) return 0u;
  const int nx = ((x0 + w - 1) >> 2) - (x0 >> 2) + 1;
  const int ny = ((y0 + h - 1) >> 2) - (y0 >> 2) + 1;
  return (uint32_t)(nx * ny);
}

// ---------------------------------------------------------------------------------
// 1. per-Gaussian rectangle and depth bucket (rasterizer.py:36-51, 84-94;
//    renderer.py:63-75 for the radius-cap statistic).
__global__ __launch_bounds__(kPrepBlock) void bin_prep_kernel(int64_t n, const float* __restrict__ means2d,
                                                              const float* __restrict__ radii,
                                                              const uint8_t* __restrict__ valid,
                                                              const float* __restrict__ depths, int W, int H,
                                                              uint32_t* __restrict__ dkey, uint2* __restrict__ rect,
                                                              uint32_t* __restrict__ blkstat) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  bool cap_violation = false, negative = false;
  if (i < n) {
    const float mx = means2d[2 * i], my = means2d[2 * i + 1], r = radii[i];
    const float wm1 = (float)(W - 1), hm1 = (float)(H - 1);
    const float minx = jmin(jmax(mx - r, 0.0f), wm1);
    const float maxx = jmin(jmax(mx + r, 0.0f), wm1);
    const float miny = jmin(jmax(my - r, 0.0f), hm1);
    const float maxy = jmin(jmax(my + r, 0.0f), hm1);
    // floor(x/16) of values in [0, W-1] (NaN only for Gaussians that are invalid).
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
  __shared__ uint32_t wcnt[2][kPrepBlock / 64];
  const uint32_t capc = (uint32_t)__popcll(__ballot(cap_violation));
  const uint32_t negc = (uint32_t)__popcll(__ballot(negative));
  if ((threadIdx.x & 63) == 0) {
    wcnt[0][threadIdx.x >> 6] = capc;
    wcnt[1][threadIdx.x >> 6] = negc;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    uint32_t s = 0;
    for (int k = 0; k < kPrepBlock / 64; ++k) s += wcnt[threadIdx.x][k];
    blkstat[2 * (int64_t)blockIdx.x + threadIdx.x] = s;
  }
}

// ---------------------------------------------------------------------------------
// Device-wide exclusive scan of uint32 (3 phases, no inter-block waiting).
struct LoadPlain {
  const uint32_t* p;
  __device__ uint32_t operator()(int64_t i) const { return p[i]; }
};
// Number of superblocks met by the Gaussian at depth-sorted position i.
struct LoadSortedSB {
  const uint32_t* order;
  const uint2* rect;
  int64_t n;
  __device__ uint32_t operator()(int64_t i) const {
    const uint32_t g = order[i];
    if ((int64_t)g >= n) return 0u;  // unreachable for a permutation; keeps reads in bounds
    return sb_count(rect[g]);
  }
};
// Number of chunks of superblock i's list.
struct LoadChunks {
  const int32_t* sb_ranges;
  __device__ uint32_t operator()(int64_t i) const {
    const int len = sb_ranges[i + 1] - sb_ranges[i];
    return (uint32_t)((len + kChunk - 1) / kChunk);
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

// Exclusive scan of one value per thread over a 256-thread block; the block total
// is returned through *total.
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

// Blocked layout: thread t owns elements [t*16, t*16+16) of the block's tile, so the
// per-thread sums compose into an exclusive scan in element order.  out[n] receives
// the grand total when write_total is set (out has n+1 elements then).
template <class Load, class Out>
__global__ __launch_bounds__(kScanBlock) void scan_down_kernel(Load load, int64_t n,
                                                               const uint32_t* __restrict__ partial, Out* out,
                                                               const uint32_t* __restrict__ total) {
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
    if (i < n) out[i] = (Out)run;
    run += v[k];
  }
  if (total != nullptr && blockIdx.x == 0 && threadIdx.x == 0) out[n] = (Out)(*total);
}

// ---------------------------------------------------------------------------------
// Stable LSD radix pass on a 7-bit digit at `shift`.  Grid = G single-wave
// workgroups; workgroup g owns keys [g*chunk, min(n,(g+1)*chunk)).  n is
// min(*n_dev, cap) when n_dev is given (device-resident count), else n_static.
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
// 3. (superblock, id) pairs of the Gaussian at depth-sorted position p, at off[p].
__global__ __launch_bounds__(256) void sb_pairs_kernel(int64_t n, const uint32_t* __restrict__ order,
                                                       const uint2* __restrict__ rect,
                                                       const uint32_t* __restrict__ off, int64_t pcap, int SX,
                                                       uint32_t* __restrict__ pkey, uint32_t* __restrict__ pval) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const uint32_t g = order[p];
  if ((int64_t)g >= n) return;
  int x0, y0, w, h;
  unpack_rect(rect[g], x0, y0, w, h);
  if (w == 0 || h == 0) return;
  int64_t o = off[p];
  for (int sy = y0 >> 2; sy <= (y0 + h - 1) >> 2; ++sy)
    for (int sx = x0 >> 2; sx <= (x0 + w - 1) >> 2; ++sx, ++o)
      if (o < pcap) {
        pkey[o] = (uint32_t)(sy * SX + sx);
        pval[o] = g;
      }
}

// ranges[t] = first index with key >= t (searchsorted-left), ranges[T] = count.
// Fixed grid, grid-stride over the device-resident count.
__global__ __launch_bounds__(256) void ranges_kernel(const uint32_t* __restrict__ keys,
                                                     const uint32_t* __restrict__ n_dev, int64_t cap, int T,
                                                     int32_t* __restrict__ ranges) {
  int64_t M = *n_dev;
  if (M > cap) M = cap;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i <= M; i += stride) {
    int64_t tp = i > 0 ? (int64_t)keys[i - 1] : -1;
    int64_t tc = i < M ? (int64_t)keys[i] : (int64_t)T;
    if (tp < -1) tp = -1;
    if (tc > T) tc = T;
    for (int64_t t = tp + 1; t <= tc; ++t) ranges[t] = (int32_t)i;
  }
}

// chunk c of superblock s covers its list positions [c*256, c*256+256).
__global__ __launch_bounds__(256) void chunk_map_kernel(int S, const uint32_t* __restrict__ chunk_base,
                                                        int64_t cmax, uint32_t* __restrict__ chunk_sb) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= S) return;
  for (uint32_t c = chunk_base[s]; c < chunk_base[s + 1] && c < (uint64_t)cmax; ++c) chunk_sb[c] = (uint32_t)s;
}

// One wave's view of a 64-Gaussian step of a chunk: lane masks of the 4 tile
// columns and 4 tile rows of the superblock met by each lane's rectangle.
struct StepMasks {
  uint64_t col[kSB], row[kSB];
};

__device__ inline StepMasks step_masks(bool act, int x0, int y0, int w, int h, int sx, int sy) {
  StepMasks m;
#pragma unroll
  for (int k = 0; k < kSB; ++k) {
    const int tx = sx * kSB + k, ty = sy * kSB + k;
    m.col[k] = __ballot(act && x0 <= tx && tx < x0 + w);
    m.row[k] = __ballot(act && y0 <= ty && ty < y0 + h);
  }
  return m;
}

struct ChunkSpan {
  int s, sx, sy;
  int64_t begin, end;  // positions in the superblock-sorted pair list
};

__device__ inline ChunkSpan chunk_span(uint32_t c, const uint32_t* __restrict__ chunk_sb,
                                       const uint32_t* __restrict__ chunk_base, const int32_t* __restrict__ sb_ranges,
                                       int S, int SX) {
  ChunkSpan cs;
  cs.s = min((int)chunk_sb[c], S - 1);
  cs.sx = cs.s % SX;
  cs.sy = cs.s / SX;
  const int64_t lo = sb_ranges[cs.s], hi = sb_ranges[cs.s + 1];
  cs.begin = lo + (int64_t)(c - chunk_base[cs.s]) * kChunk;
  cs.end = cs.begin + kChunk < hi ? cs.begin + kChunk : hi;
  return cs;
}

// 4a. counts per (chunk, tile of its superblock): cnt[c*16 + u], u = 4*(ty%4) + tx%4.
__global__ __launch_bounds__(256) void tile_count_kernel(const uint32_t* __restrict__ n_chunks, int64_t cmax,
                                                         const uint32_t* __restrict__ chunk_sb,
                                                         const uint32_t* __restrict__ chunk_base,
                                                         const int32_t* __restrict__ sb_ranges, int S,
                                                         const uint32_t* __restrict__ pval,
                                                         const uint2* __restrict__ rect, uint32_t n_gauss,
                                                         int SX, uint32_t* __restrict__ cnt) {
  const int lane = threadIdx.x & 63;
  const uint32_t nwaves = gridDim.x * (blockDim.x / 64);
  const uint32_t C = (uint32_t)min<int64_t>((int64_t)*n_chunks, cmax);
  for (uint32_t c = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); c < C; c += nwaves) {
    const ChunkSpan cs = chunk_span(c, chunk_sb, chunk_base, sb_ranges, S, SX);
    uint32_t mycount = 0;  // lane u < 16 accumulates tile u
    for (int64_t base = cs.begin; base < cs.end; base += 64) {
      const int64_t q = base + lane;
      bool act = q < cs.end;
      int x0 = 0, y0 = 0, w = 0, h = 0;
      const uint32_t g = act ? pval[q] : 0u;
      act = act && g < n_gauss;  // ids are < n by construction; keeps reads in bounds
      if (act) unpack_rect(rect[g], x0, y0, w, h);
      const StepMasks m = step_masks(act, x0, y0, w, h, cs.sx, cs.sy);
      uint64_t mine = 0;
#pragma unroll
      for (int u = 0; u < 16; ++u) mine = (lane == u) ? (m.col[u & 3] & m.row[u >> 2]) : mine;
      mycount += (uint32_t)__popcll(mine);
    }
    if (lane < 16) cnt[(int64_t)c * 16 + lane] = mycount;
  }
}

// 4b. per tile: total over the chunks of its superblock.
__global__ __launch_bounds__(256) void tile_total_kernel(int T, int TX, int SX, int64_t cmax,
                                                         const uint32_t* __restrict__ chunk_base,
                                                         const uint32_t* __restrict__ cnt,
                                                         uint32_t* __restrict__ tot) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const int tx = t % TX, ty = t / TX;
  const int s = (ty >> 2) * SX + (tx >> 2), u = (ty & 3) * 4 + (tx & 3);
  uint32_t acc = 0;
  const uint32_t ce = (uint32_t)min<int64_t>(chunk_base[s + 1], cmax);
  for (uint32_t c = chunk_base[s]; c < ce; ++c) acc += cnt[(int64_t)c * 16 + u];
  tot[t] = acc;
}

// 4c. per tile: starting offset of each chunk's entries, in place of the counts.
__global__ __launch_bounds__(256) void tile_offsets_kernel(int T, int TX, int SX, int64_t cmax,
                                                           const uint32_t* __restrict__ chunk_base,
                                                           const int32_t* __restrict__ ranges,
                                                           uint32_t* __restrict__ cnt) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const int tx = t % TX, ty = t / TX;
  const int s = (ty >> 2) * SX + (tx >> 2), u = (ty & 3) * 4 + (tx & 3);
  uint32_t run = (uint32_t)ranges[t];
  const uint32_t ce = (uint32_t)min<int64_t>(chunk_base[s + 1], cmax);
  for (uint32_t c = chunk_base[s]; c < ce; ++c) {
    const uint32_t k = cnt[(int64_t)c * 16 + u];
    cnt[(int64_t)c * 16 + u] = run;
    run += k;
  }
}

// 4d. write every entry: tile t's entries from chunk c start at off[c*16+u]; within a
// step, lane L's entry in tile u is preceded by popcount(mask_u & lanes-below-L).
__global__ __launch_bounds__(256) void tile_write_kernel(const uint32_t* __restrict__ n_chunks, int64_t cmax,
                                                         const uint32_t* __restrict__ chunk_sb,
                                                         const uint32_t* __restrict__ chunk_base,
                                                         const int32_t* __restrict__ sb_ranges, int S,
                                                         const uint32_t* __restrict__ pval,
                                                         const uint2* __restrict__ rect, uint32_t n_gauss,
                                                         int SX, int TX, const uint32_t* __restrict__ off,
                                                         int64_t cap,
                                                         int32_t* __restrict__ out_gid,
                                                         int32_t* __restrict__ out_tile) {
  __shared__ uint64_t smask[4][16];
  __shared__ uint32_t sbase[4][16];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint32_t nwaves = gridDim.x * (blockDim.x / 64);
  const uint32_t C = (uint32_t)min<int64_t>((int64_t)*n_chunks, cmax);
  const uint64_t lt = lanemask_lt();
  for (uint32_t c = blockIdx.x * (blockDim.x / 64) + wid; c < C; c += nwaves) {
    const ChunkSpan cs = chunk_span(c, chunk_sb, chunk_base, sb_ranges, S, SX);
    if (lane < 16) sbase[wid][lane] = off[(int64_t)c * 16 + lane];
    for (int64_t base = cs.begin; base < cs.end; base += 64) {
      const int64_t q = base + lane;
      bool act = q < cs.end;
      int x0 = 0, y0 = 0, w = 0, h = 0;
      const uint32_t g = act ? pval[q] : 0u;
      act = act && g < n_gauss;  // ids are < n by construction; keeps reads in bounds
      if (act) unpack_rect(rect[g], x0, y0, w, h);
      const StepMasks m = step_masks(act, x0, y0, w, h, cs.sx, cs.sy);
      uint64_t mine = 0;
#pragma unroll
      for (int u = 0; u < 16; ++u) mine = (lane == u) ? (m.col[u & 3] & m.row[u >> 2]) : mine;
      if (lane < 16) smask[wid][lane] = mine;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (act) {
        const int ux0 = max(x0, cs.sx * kSB), ux1 = min(x0 + w, cs.sx * kSB + kSB);
        const int uy0 = max(y0, cs.sy * kSB), uy1 = min(y0 + h, cs.sy * kSB + kSB);
        for (int ty = uy0; ty < uy1; ++ty)
          for (int tx = ux0; tx < ux1; ++tx) {
            const int u = (ty - cs.sy * kSB) * kSB + (tx - cs.sx * kSB);
            const int64_t dst = (int64_t)sbase[wid][u] + __popcll(smask[wid][u] & lt);
            if (dst < cap) {
              out_gid[dst] = (int32_t)g;
              if (out_tile) out_tile[dst] = ty * TX + tx;
            }
          }
      }
      __builtin_amdgcn_wave_barrier();
      if (lane < 16) sbase[wid][lane] += (uint32_t)__popcll(mine);
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

// 5. renderer.py:76-89 from the tile ranges, plus the per-block prep counts.
__global__ __launch_bounds__(256) void stats_kernel(const int32_t* __restrict__ ranges, int T,
                                                    const uint32_t* __restrict__ blkstat, int nblk, int64_t cap,
                                                    int32_t* __restrict__ stats) {
  int mx = 0;
  int64_t ot = 0, oi = 0, tt = 0, ti = 0, cv = 0, ng = 0;
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const int c = ranges[t + 1] - ranges[t];
    mx = max(mx, c);
    ot += c > kBlock;
    oi += c > kBlock ? c - kBlock : 0;
    tt += c > kMaxTileEntries;
    ti += c > kMaxTileEntries ? c - kMaxTileEntries : 0;
  }
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    cv += blkstat[2 * b];
    ng += blkstat[2 * b + 1];
  }
  __shared__ int64_t red[6][256];
  __shared__ int rmax[256];
  rmax[threadIdx.x] = mx;
  red[0][threadIdx.x] = ot;
  red[1][threadIdx.x] = oi;
  red[2][threadIdx.x] = tt;
  red[3][threadIdx.x] = ti;
  red[4][threadIdx.x] = cv;
  red[5][threadIdx.x] = ng;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      rmax[threadIdx.x] = max(rmax[threadIdx.x], rmax[threadIdx.x + o]);
      for (int k = 0; k < 6; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    for (int k = 0; k < GS_NUM_STATS; ++k) stats[k] = 0;
    const int64_t m = ranges[T];
    stats[GS_STAT_N_INTERACTIONS] = (int32_t)m;
    stats[GS_STAT_MAX_PER_TILE] = rmax[0];
    stats[GS_STAT_OVERFLOW_TILES] = (int32_t)red[0][0];
    stats[GS_STAT_OVERFLOW_INTERACTIONS] = (int32_t)red[1][0];
    stats[GS_STAT_TRUNCATED_TILES] = (int32_t)red[2][0];
    stats[GS_STAT_TRUNCATED_INTERACTIONS] = (int32_t)red[3][0];
    stats[GS_STAT_RADIUS_CAP_VIOLATIONS] = (int32_t)red[4][0];
    stats[GS_STAT_NEGATIVE_DEPTH] = (int32_t)red[5][0];
    stats[GS_STAT_CAPACITY_EXCEEDED] = m > cap ? 1 : 0;
  }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------------
struct BinPlan {
  int64_t n, cap, pcap, cmax;
  int T, TX, TY, SX, SY, S;
  int G_d, G_p;  // radix grids for the depth sort and the superblock sort
  int sb_passes;
  int nblk_prep;
  size_t o_dkey, o_rect, o_ka, o_va, o_kb, o_vb, o_off, o_part, o_table, o_scal, o_pk0, o_pv0, o_pk1, o_pv1,
      o_sbr, o_cbase, o_csb, o_cnt, o_tot, o_blk, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

BinPlan make_plan(int64_t n, int width, int height, int64_t capacity) {
  BinPlan P;
  P.n = n;
  P.cap = capacity > 0 ? capacity : 256 * (n > 2 ? n : 2);
  P.TX = (width + kTile - 1) / kTile;
  P.TY = (height + kTile - 1) / kTile;
  P.T = P.TX * P.TY;
  P.SX = (P.TX + kSB - 1) / kSB;
  P.SY = (P.TY + kSB - 1) / kSB;
  P.S = P.SX * P.SY;
  int bits = 1;
  while ((1 << bits) < P.S) ++bits;
  P.sb_passes = (bits + kRadixBits - 1) / kRadixBits;
  const int64_t nn = std::max<int64_t>(n, 1);
  P.pcap = kSBMax * nn;
  P.cmax = (P.pcap + kChunk - 1) / kChunk + P.S;
  P.G_d = (int)std::min<int64_t>(4096, std::max<int64_t>(1, (nn + 1023) / 1024));
  P.G_p = (int)std::min<int64_t>(4096, std::max<int64_t>(1, (2 * nn + 1023) / 1024));
  P.nblk_prep = div_up(nn, kPrepBlock);
  const int64_t tbl = (int64_t)kRadixBins * std::max(P.G_d, P.G_p);
  const int64_t scan_max = std::max<int64_t>({nn, tbl, (int64_t)P.T, (int64_t)P.S});
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  P.o_dkey = take(nn * 4);
  P.o_rect = take(nn * 8);
  P.o_ka = take(nn * 4);
  P.o_va = take(nn * 4);
  P.o_kb = take(nn * 4);
  P.o_vb = take(nn * 4);
  P.o_off = take((nn + 1) * 4);
  P.o_part = take((size_t)div_up(scan_max, kScanTile) * 4 + 64);
  P.o_table = take((size_t)tbl * 4);
  P.o_scal = take(256);  // device scalars: [0] pairs, [1] chunks
  P.o_pk0 = take((size_t)P.pcap * 4);
  P.o_pv0 = take((size_t)P.pcap * 4);
  P.o_pk1 = take((size_t)P.pcap * 4);
  P.o_pv1 = take((size_t)P.pcap * 4);
  P.o_sbr = take(((size_t)P.S + 1) * 4);
  P.o_cbase = take(((size_t)P.S + 1) * 4);
  P.o_csb = take((size_t)P.cmax * 4);
  P.o_cnt = take((size_t)P.cmax * 16 * 4);
  P.o_tot = take((size_t)P.T * 4);
  P.o_blk = take((size_t)P.nblk_prep * 2 * 4);
  P.total = o;
  return P;
}

template <class Load, class Out>
int run_scan(hipStream_t s, Load load, int64_t n, uint32_t* partial, Out* out, uint32_t* total) {
  const int nb = div_up(std::max<int64_t>(n, 1), kScanTile);
  if (nb > kMaxScanPartials) {
    set_error("gs_bin: scan of %lld elements exceeds the supported size", (long long)n);
    return GS_ERR_INVALID;
  }
  hipLaunchKernelGGL(scan_reduce_kernel<Load>, dim3(nb), dim3(kScanBlock), 0, s, load, n, partial);
  GS_LAUNCH_CHECK("scan_reduce_kernel");
  hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(kScanBlock), 0, s, partial, nb, total);
  GS_LAUNCH_CHECK("scan_partials_kernel");
  hipLaunchKernelGGL((scan_down_kernel<Load, Out>), dim3(nb), dim3(kScanBlock), 0, s, load, n, partial, out,
                     (const uint32_t*)total);
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
  GS_REQUIRE(n >= 0 && n <= ((int64_t)1 << 26), "gs_bin: n must be in [0, 2^26] (got %lld)", (long long)n);
  GS_REQUIRE(width > 0 && height > 0 && width <= 65535 * kTile && height <= 65535 * kTile,
             "gs_bin: bad image size %dx%d", width, height);
  const BinPlan P = make_plan(n, width, height, capacity);
  GS_REQUIRE(P.cap < ((int64_t)1 << 31), "gs_bin: capacity %lld too large", (long long)P.cap);
  GS_REQUIRE(P.sb_passes <= 2, "gs_bin: %d tiles exceed the supported 16384 superblocks", P.T);
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
  uint32_t* scal = (uint32_t*)(ws + P.o_scal);
  uint32_t* pk0 = (uint32_t*)(ws + P.o_pk0);
  uint32_t* pv0 = (uint32_t*)(ws + P.o_pv0);
  uint32_t* pk1 = (uint32_t*)(ws + P.o_pk1);
  uint32_t* pv1 = (uint32_t*)(ws + P.o_pv1);
  int32_t* sbr = (int32_t*)(ws + P.o_sbr);
  uint32_t* cbase = (uint32_t*)(ws + P.o_cbase);
  uint32_t* csb = (uint32_t*)(ws + P.o_csb);
  uint32_t* cnt = (uint32_t*)(ws + P.o_cnt);
  uint32_t* tot = (uint32_t*)(ws + P.o_tot);
  uint32_t* blk = (uint32_t*)(ws + P.o_blk);
  uint32_t* n_pairs = scal + 0;
  uint32_t* n_chunks = scal + 1;

  if (n == 0) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, s, stats, (int64_t)GS_NUM_STATS, 0);
    GS_LAUNCH_CHECK("fill_i32_kernel");
    hipLaunchKernelGGL(fill_i32_kernel, dim3(div_up(P.T + 1, 256)), dim3(256), 0, s, ranges, (int64_t)P.T + 1, 0);
    GS_LAUNCH_CHECK("fill_i32_kernel");
    return GS_OK;
  }
  // 1. prep
  hipLaunchKernelGGL(bin_prep_kernel, dim3(P.nblk_prep), dim3(kPrepBlock), 0, s, n, means2d, radii, valid, depths,
                     width, height, dkey, rect, blk);
  GS_LAUNCH_CHECK("bin_prep_kernel");
  // 2. stable depth sort of Gaussian ids (13-bit bucket: 7 + 6 bits)
  int rc = radix_pass(s, dkey, nullptr, kb, vb, nullptr, n, n, 0, P.G_d, table, part);
  if (rc != GS_OK) return rc;
  rc = radix_pass(s, kb, vb, ka, va, nullptr, n, n, kRadixBits, P.G_d, table, part);
  if (rc != GS_OK) return rc;
  const uint32_t* order = va;
  // 3. superblock pairs in depth order, stably sorted by superblock
  rc = run_scan(s, LoadSortedSB{order, rect, n}, n, part, off, n_pairs);
  if (rc != GS_OK) return rc;
  hipLaunchKernelGGL(sb_pairs_kernel, dim3(div_up(n, 256)), dim3(256), 0, s, n, order, rect, off, P.pcap, P.SX, pk0,
                     pv0);
  GS_LAUNCH_CHECK("sb_pairs_kernel");
  uint32_t* sbkey = pk0;
  uint32_t* sbval = pv0;
  if (P.sb_passes >= 1) {
    rc = radix_pass(s, pk0, pv0, pk1, pv1, n_pairs, 0, P.pcap, 0, P.G_p, table, part);
    if (rc != GS_OK) return rc;
    sbkey = pk1;
    sbval = pv1;
  }
  if (P.sb_passes == 2) {
    rc = radix_pass(s, pk1, pv1, pk0, pv0, n_pairs, 0, P.pcap, kRadixBits, P.G_p, table, part);
    if (rc != GS_OK) return rc;
    sbkey = pk0;
    sbval = pv0;
  }
  hipLaunchKernelGGL(ranges_kernel, dim3(std::min(2048, div_up(P.pcap + 1, 256))), dim3(256), 0, s, sbkey, n_pairs,
                     P.pcap, P.S, sbr);
  GS_LAUNCH_CHECK("ranges_kernel");
  // 4. tile pass
  rc = run_scan(s, LoadChunks{sbr}, P.S, part, cbase, n_chunks);
  if (rc != GS_OK) return rc;
  hipLaunchKernelGGL(chunk_map_kernel, dim3(div_up(P.S, 256)), dim3(256), 0, s, P.S, cbase, P.cmax, csb);
  GS_LAUNCH_CHECK("chunk_map_kernel");
  const int pass_blocks = 2048;
  hipLaunchKernelGGL(tile_count_kernel, dim3(pass_blocks), dim3(256), 0, s, n_chunks, P.cmax, csb, cbase, sbr, P.S,
                     sbval, rect, (uint32_t)n, P.SX, cnt);
  GS_LAUNCH_CHECK("tile_count_kernel");
  hipLaunchKernelGGL(tile_total_kernel, dim3(div_up(P.T, 256)), dim3(256), 0, s, P.T, P.TX, P.SX, P.cmax, cbase, cnt,
                     tot);
  GS_LAUNCH_CHECK("tile_total_kernel");
  rc = run_scan(s, LoadPlain{tot}, P.T, part, ranges, part + div_up(P.T, kScanTile));
  if (rc != GS_OK) return rc;
  hipLaunchKernelGGL(tile_offsets_kernel, dim3(div_up(P.T, 256)), dim3(256), 0, s, P.T, P.TX, P.SX, P.cmax, cbase,
                     ranges, cnt);
  GS_LAUNCH_CHECK("tile_offsets_kernel");
  hipLaunchKernelGGL(tile_write_kernel, dim3(pass_blocks), dim3(256), 0, s, n_chunks, P.cmax, csb, cbase, sbr, P.S,
                     sbval, rect, (uint32_t)n, P.SX, P.TX, cnt, P.cap, sorted_gids, sorted_tiles);
  GS_LAUNCH_CHECK("tile_write_kernel");
  // 5. stats
  hipLaunchKernelGGL(stats_kernel, dim3(1), dim3(256), 0, s, ranges, P.T, blk, P.nblk_prep, P.cap, stats);
  GS_LAUNCH_CHECK("stats_kernel");
  return GS_OK;
}

// Same boundary rule on a caller-provided sorted array that may hold -1 (negative
// depth) and T (sentinel) entries.
namespace gs {
namespace {
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
}  // namespace
}  // namespace gs

extern "C" int gs_tile_ranges(void* stream, const int32_t* sorted_tiles, int64_t length, int num_tiles,
                              int32_t* ranges) {
  GS_REQUIRE(length >= 0 && num_tiles >= 0, "gs_tile_ranges: bad sizes");
  GS_REQUIRE(ranges != nullptr && (length == 0 || sorted_tiles != nullptr), "gs_tile_ranges: NULL argument");
  hipLaunchKernelGGL(ranges_any_kernel, dim3(std::min<int64_t>(2048, div_up(length + 1, 256))), dim3(256), 0,
                     (hipStream_t)stream, sorted_tiles, length, num_tiles, ranges);
  GS_LAUNCH_CHECK("ranges_any_kernel");
  return GS_OK;
}
