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
//                      bucket, packed with the id into one 64-bit word; per-block
//                      counts of radius-cap violations and negative depths; histogram
//                      of the first radix digit of the bucket.
//   2. depth sort      stable LSD radix sort of the packed words by depth bucket (two
//                      7-bit passes)  -> Gaussians in (bucket, id) order.
//   3. superblocks     every Gaussian meets at most 5x5 "superblocks" of 4x4 tiles;
//                      its (superblock, packed word) pairs are written in depth order
//                      and stably sorted by superblock (two 7-bit passes) -> per
//                      superblock the list of Gaussians touching it, in (bucket, id)
//                      order.  Carrying the rectangle in the sorted word keeps every
//                      later read coalesced.
//   4. tile pass       a superblock's list is cut into chunks of 256 Gaussians; a wave
//                      takes a chunk 64 Gaussians at a time and forms 4 column and 4
//                      row lane masks with ballots, so for each of the 16 tiles it
//                      knows which lanes hit it.  A counting sweep gives per (chunk,
//                      tile) counts and tile totals, one scan gives the tile ranges,
//                      and a writing sweep stores each entry's id at
//                      range + counts of earlier chunks + popcount(mask & lanes-below)
//                      -- stable by construction.
//   5. stats           the renderer's health extras, computed with the range scan.
//
// Radix passes use one wave per workgroup over a contiguous key range (in-wave rank
// with ballot "match any"), a per-digit spine scan across workgroups, and no
// inter-workgroup waiting.  There are no same-address atomics.
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
constexpr int kPrepPer = 4;                         // Gaussians per bin_prep thread
constexpr int kPrepSpan = kPrepBlock * kPrepPer;    // = depth-sort workgroup range
constexpr int kBig = 1024;                          // single-block scan kernels

__device__ inline uint64_t lanemask_lt() {
  const unsigned lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Packed Gaussian word: id (26 bits) | tminx (12) | tminy (12) | w-1 (4) | h-1 (4) |
// has-entries (1).
struct Packed {
  uint32_t gid;
  int x0, y0, w, h;  // w = h = 0 when the Gaussian meets no tile
};
__device__ inline uint64_t pack(uint32_t gid, int x0, int y0, int w, int h) {
  uint64_t v = gid;
  if (w > 0 && h > 0)
    v |= ((uint64_t)x0 << 26) | ((uint64_t)y0 << 38) | ((uint64_t)(w - 1) << 50) | ((uint64_t)(h - 1) << 54) |
         (1ull << 58);
  return v;
}
__device__ inline Packed unpack(uint64_t v) {
  Packed p;
  p.gid = (uint32_t)(v & 0x3FFFFFFull);
  const bool has = (v >> 58) & 1;
  p.x0 = (int)((v >> 26) & 0xFFF);
  p.y0 = (int)((v >> 38) & 0xFFF);
  p.w = has ? (int)((v >> 50) & 0xF) + 1 : 0;
  p.h = has ? (int)((v >> 54) & 0xF) + 1 : 0;
  return p;
}
__device__ inline uint32_t sb_count(const Packed& p) {
  if (p.w == 0) return 0u;
  const int nx = ((p.x0 + p.w - 1) >> 2) - (p.x0 >> 2) + 1;
  const int ny = ((p.y0 + p.h - 1) >> 2) - (p.y0 >> 2) + 1;
  return (uint32_t)(nx * ny);
}

// ---------------------------------------------------------------------------------
// 1. per-Gaussian rectangle and depth bucket (rasterizer.py:36-51, 84-94;
//    renderer.py:63-75 for the radius-cap statistic).  Block b handles Gaussians
//    [b*1024, b*1024+1024), the same range as depth-sort workgroup b, and writes that
//    workgroup's histogram of the first radix digit.
__global__ __launch_bounds__(kPrepBlock) void bin_prep_kernel(int64_t n, const float* __restrict__ means2d,
                                                              const float* __restrict__ radii,
                                                              const uint8_t* __restrict__ valid,
                                                              const float* __restrict__ depths, int W, int H, int G,
                                                              uint32_t* __restrict__ dkey, uint64_t* __restrict__ word,
                                                              uint32_t* __restrict__ table,
                                                              uint32_t* __restrict__ blkstat) {
  __shared__ uint32_t hist[kRadixBins];
  __shared__ uint32_t wcnt[2][kPrepBlock / 64];
  for (int d = threadIdx.x; d < kRadixBins; d += kPrepBlock) hist[d] = 0;
  __syncthreads();
  uint32_t capc = 0, negc = 0;
  for (int r = 0; r < kPrepPer; ++r) {
    const int64_t i = (int64_t)blockIdx.x * kPrepSpan + r * kPrepBlock + threadIdx.x;
    bool cap_violation = false, negative = false;
    if (i < n) {
      const float mx = means2d[2 * i], my = means2d[2 * i + 1], rr = radii[i];
      const float wm1 = (float)(W - 1), hm1 = (float)(H - 1);
      const float minx = jmin(jmax(mx - rr, 0.0f), wm1);
      const float maxx = jmin(jmax(mx + rr, 0.0f), wm1);
      const float miny = jmin(jmax(my - rr, 0.0f), hm1);
      const float maxy = jmin(jmax(my + rr, 0.0f), hm1);
      // floor(x/16) of values in [0, W-1] (NaN only for Gaussians that are invalid).
      const int tminx = (int)floorf(minx / 16.0f), tmaxx = (int)floorf(maxx / 16.0f);
      const int tminy = (int)floorf(miny / 16.0f), tmaxy = (int)floorf(maxy / 16.0f);
      const bool on_screen = (mx + rr > 0.0f) && (mx - rr < (float)W) && (my + rr > 0.0f) && (my - rr < (float)H);
      const bool proj_valid = valid[i] != 0;
      const bool v = proj_valid && on_screen && (tmaxx >= tminx) && (tmaxy >= tminy);
      const int spanx = tmaxx - tminx + 1, spany = tmaxy - tminy + 1;
      cap_violation = proj_valid && on_screen && (spanx > kOffset || spany > kOffset);
      const uint32_t zb = float_to_bits(depths[i]);
      negative = (zb >> 31) != 0;
      uint32_t key = kDepthBinEmpty;
      int w = 0, h = 0;
      if (v) {
        w = spanx < kOffset ? spanx : kOffset;
        h = spany < kOffset ? spany : kOffset;
        // v implies depth > 0.01, so the 13-bit bucket is in [3848, 8191].
        key = (zb >> (31 - kDepthBits)) - kDepthBucketLo;
      }
      dkey[i] = key;
      word[i] = pack((uint32_t)i, v ? tminx : 0, v ? tminy : 0, w, h);
      atomicAdd(&hist[key & (kRadixBins - 1)], 1u);
    }
    capc += (uint32_t)__popcll(__ballot(cap_violation));
    negc += (uint32_t)__popcll(__ballot(negative));
  }
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
  for (int d = threadIdx.x; d < kRadixBins; d += kPrepBlock) table[(int64_t)d * G + blockIdx.x] = hist[d];
}

// ---------------------------------------------------------------------------------
// Device-wide exclusive scan of uint32 (3 phases, no inter-block waiting).
struct LoadPlain {
  const uint32_t* p;
  __device__ uint32_t operator()(int64_t i) const { return p[i]; }
};
// Number of superblocks met by the Gaussian at depth-sorted position i.
struct LoadSortedSB {
  const uint64_t* word;
  __device__ uint32_t operator()(int64_t i) const { return sb_count(unpack(word[i])); }
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

// Exclusive scan of one value per thread over a block of NT threads; the block total
// is returned through *total.
template <int NT>
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t* total) {
  constexpr int NW = NT / 64;
  __shared__ uint32_t wsum[NW];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint32_t inc = wave_incl_scan(v);
  if (lane == 63) wsum[wid] = inc;
  __syncthreads();
  uint32_t wbase = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < NW; ++k) {
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
  block_excl_scan<kScanBlock>(s, &tot);
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
    const uint32_t ex = block_excl_scan<kScanBlock>(v, &tot);
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
// the grand total when total is given (out has n+1 elements then).
template <class Load>
__global__ __launch_bounds__(kScanBlock) void scan_down_kernel(Load load, int64_t n,
                                                               const uint32_t* __restrict__ partial,
                                                               uint32_t* __restrict__ out,
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
  uint32_t run = partial[blockIdx.x] + block_excl_scan<kScanBlock>(s, &tot);
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    const int64_t i = base + k;
    if (i < n) out[i] = run;
    run += v[k];
  }
  if (total != nullptr && blockIdx.x == 0 && threadIdx.x == 0) out[n] = *total;
}

// ---------------------------------------------------------------------------------
// Stable LSD radix pass on a 7-bit digit at `shift`, keys u32 + values u64.
// Workgroup g (one wave) owns keys [g*chunk, min(n,(g+1)*chunk)); chunk is fixed when
// given, else derived from G.  n is min(*n_dev, cap) when n_dev is given.
__device__ inline void pass_range(const uint32_t* n_dev, int64_t n_static, int64_t cap, int G, int fixed_chunk,
                                  int64_t& begin, int64_t& end, int64_t* n_out = nullptr) {
  int64_t n = n_static;
  if (n_dev != nullptr) {
    n = (int64_t)(*n_dev);
    if (n > cap) n = cap;
  }
  int64_t chunk = fixed_chunk;
  if (chunk == 0) {
    chunk = (n + G - 1) / G;
    chunk = (chunk + 63) & ~(int64_t)63;
  }
  begin = (int64_t)blockIdx.x * chunk;
  end = begin + chunk;
  if (end > n) end = n;
  if (n_out) *n_out = n;
}

__global__ __launch_bounds__(64) void radix_upsweep_kernel(const uint32_t* __restrict__ keys,
                                                           const uint32_t* __restrict__ n_dev,
                                                           int64_t n_static, int64_t cap, int shift, int G,
                                                           int fixed_chunk, uint32_t* __restrict__ table) {
  __shared__ uint32_t hist[kRadixBins];
  const int lane = threadIdx.x;
  for (int d = lane; d < kRadixBins; d += 64) hist[d] = 0;
  __syncthreads();
  int64_t begin, end;
  pass_range(n_dev, n_static, cap, G, fixed_chunk, begin, end);
  for (int64_t i = begin + lane; i < end; i += 64) atomicAdd(&hist[(keys[i] >> shift) & (kRadixBins - 1)], 1u);
  __syncthreads();
  for (int d = lane; d < kRadixBins; d += 64) table[(int64_t)d * G + blockIdx.x] = hist[d];
}

// One block per digit: exclusive scan of that digit's row of the table (over the G
// workgroups) in place, and the digit's total.
__global__ __launch_bounds__(kScanBlock) void radix_spine_kernel(uint32_t* __restrict__ table, int G,
                                                                 uint32_t* __restrict__ digit_tot) {
  const int d = blockIdx.x;
  uint32_t* row = table + (int64_t)d * G;
  const int per = (G + kScanBlock - 1) / kScanBlock;
  const int b0 = threadIdx.x * per;
  uint32_t s = 0;
  for (int k = 0; k < per; ++k)
    if (b0 + k < G) s += row[b0 + k];
  uint32_t tot;
  uint32_t run = block_excl_scan<kScanBlock>(s, &tot);
  for (int k = 0; k < per; ++k)
    if (b0 + k < G) {
      const uint32_t v = row[b0 + k];
      row[b0 + k] = run;
      run += v;
    }
  if (threadIdx.x == 0) digit_tot[d] = tot;
}

constexpr int kUnroll = 4;

__global__ __launch_bounds__(64) void radix_downsweep_kernel(
    const uint32_t* __restrict__ keys_in, const uint64_t* __restrict__ vals_in, const uint32_t* __restrict__ n_dev,
    int64_t n_static, int64_t cap, int shift, int G, int fixed_chunk, const uint32_t* __restrict__ table,
    const uint32_t* __restrict__ digit_tot, uint32_t* __restrict__ keys_out, uint64_t* __restrict__ vals_out) {
  __shared__ uint32_t cnt[kRadixBins];
  const int lane = threadIdx.x;
  {
    // digit bases: exclusive scan of the digit totals (2 digits per lane)
    const uint32_t a = digit_tot[2 * lane], b = digit_tot[2 * lane + 1];
    const uint32_t inc = wave_incl_scan(a + b);
    const uint32_t base = inc - (a + b);
    cnt[2 * lane] = base + table[(int64_t)(2 * lane) * G + blockIdx.x];
    cnt[2 * lane + 1] = base + a + table[(int64_t)(2 * lane + 1) * G + blockIdx.x];
  }
  __syncthreads();
  int64_t begin, end, n_pass;
  pass_range(n_dev, n_static, cap, G, fixed_chunk, begin, end, &n_pass);
  const uint64_t lt = lanemask_lt();
  for (int64_t base = begin; base < end; base += 64 * kUnroll) {
    uint32_t k[kUnroll];
    uint64_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * 64 + lane;
      const bool a = i < end;
      k[u] = a ? keys_in[i] : 0u;
      v[u] = a ? vals_in[i] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * 64 + lane;
      const bool a = i < end;
      const uint32_t d = (k[u] >> shift) & (kRadixBins - 1);
      uint64_t m = __ballot(a);
#pragma unroll
      for (int bb = 0; bb < kRadixBits; ++bb) {
        const bool bit = (d >> bb) & 1u;
        const uint64_t bm = __ballot(bit);
        m &= bit ? bm : ~bm;
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
        keys_out[dst] = k[u];
        vals_out[dst] = v[u];
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// 3. (superblock, word) pairs of the Gaussian at depth-sorted position p, at off[p].
__global__ __launch_bounds__(256) void sb_pairs_kernel(int64_t n, const uint64_t* __restrict__ word,
                                                       const uint32_t* __restrict__ off, int64_t pcap, int SX,
                                                       uint32_t* __restrict__ pkey, uint64_t* __restrict__ pval) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  const uint64_t wv = word[p];
  const Packed g = unpack(wv);
  if (g.w == 0) return;
  int64_t o = off[p];
  for (int sy = g.y0 >> 2; sy <= (g.y0 + g.h - 1) >> 2; ++sy)
    for (int sx = g.x0 >> 2; sx <= (g.x0 + g.w - 1) >> 2; ++sx, ++o)
      if (o < pcap) {
        pkey[o] = (uint32_t)(sy * SX + sx);
        pval[o] = wv;
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

// One block: chunk count per superblock -> exclusive scan -> chunk_base[S+1] and
// the chunk -> superblock map; also clears the tile totals.
__global__ __launch_bounds__(kBig) void chunks_kernel(int S, const int32_t* __restrict__ sb_ranges, int64_t cmax,
                                                      uint32_t* __restrict__ chunk_base,
                                                      uint32_t* __restrict__ chunk_sb, uint32_t* __restrict__ n_chunks,
                                                      int T, uint32_t* __restrict__ tot) {
  for (int t = threadIdx.x; t < T; t += kBig) tot[t] = 0;
  __shared__ uint32_t carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int s0 = 0; s0 < S; s0 += kBig) {
    const int s = s0 + threadIdx.x;
    uint32_t nc = 0;
    if (s < S) nc = (uint32_t)((sb_ranges[s + 1] - sb_ranges[s] + kChunk - 1) / kChunk);
    uint32_t sum;
    const uint32_t ex = block_excl_scan<kBig>(nc, &sum);
    const uint32_t c0 = carry + ex;
    if (s < S) {
      chunk_base[s] = c0;
      for (uint32_t c = c0; c < c0 + nc && (int64_t)c < cmax; ++c) chunk_sb[c] = (uint32_t)s;
    }
    __syncthreads();
    if (threadIdx.x == 0) carry += sum;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    chunk_base[S] = carry;
    *n_chunks = carry;
  }
}

// One wave's view of a 64-Gaussian step of a chunk: lane masks of the 4 tile columns
// and 4 tile rows of the superblock met by each lane's rectangle.
struct StepMasks {
  uint64_t col[kSB], row[kSB];
};

__device__ inline StepMasks step_masks(bool act, const Packed& g, int sx, int sy) {
  StepMasks m;
#pragma unroll
  for (int k = 0; k < kSB; ++k) {
    const int tx = sx * kSB + k, ty = sy * kSB + k;
    m.col[k] = __ballot(act && g.x0 <= tx && tx < g.x0 + g.w);
    m.row[k] = __ballot(act && g.y0 <= ty && ty < g.y0 + g.h);
  }
  return m;
}

struct ChunkSpan {
  int s, sx, sy;
  uint32_t first;      // first chunk of the superblock
  int64_t begin, end;  // positions in the superblock-sorted pair list
};

__device__ inline ChunkSpan chunk_span(uint32_t c, const uint32_t* __restrict__ chunk_sb,
                                       const uint32_t* __restrict__ chunk_base, const int32_t* __restrict__ sb_ranges,
                                       int S, int SX) {
  ChunkSpan cs;
  cs.s = min((int)chunk_sb[c], S - 1);
  cs.sx = cs.s % SX;
  cs.sy = cs.s / SX;
  cs.first = chunk_base[cs.s];
  const int64_t lo = sb_ranges[cs.s], hi = sb_ranges[cs.s + 1];
  cs.begin = lo + (int64_t)(c - cs.first) * kChunk;
  cs.end = cs.begin + kChunk < hi ? cs.begin + kChunk : hi;
  return cs;
}

// tile u of superblock (sx, sy), u = 4*(ty%4) + tx%4, or -1 outside the image
__device__ inline int tile_of(int sx, int sy, int u, int TX, int TY) {
  const int tx = sx * kSB + (u & 3), ty = sy * kSB + (u >> 2);
  return (tx < TX && ty < TY) ? ty * TX + tx : -1;
}

__device__ inline uint64_t lane_tile_mask(const StepMasks& m, int lane) {
  uint64_t mine = 0;
#pragma unroll
  for (int u = 0; u < 16; ++u) mine = (lane == u) ? (m.col[u & 3] & m.row[u >> 2]) : mine;
  return mine;
}

// 4a. counts per (chunk, tile of its superblock) -> cnt[c*16 + u]; tile totals by
// atomics (one per chunk and tile, distinct chunks rarely share a tile).
__global__ __launch_bounds__(256) void tile_count_kernel(const uint32_t* __restrict__ n_chunks, int64_t cmax,
                                                         const uint32_t* __restrict__ chunk_sb,
                                                         const uint32_t* __restrict__ chunk_base,
                                                         const int32_t* __restrict__ sb_ranges, int S,
                                                         const uint64_t* __restrict__ pval, int SX, int TX, int TY,
                                                         uint32_t* __restrict__ cnt, uint32_t* __restrict__ tot) {
  const int lane = threadIdx.x & 63;
  const uint32_t nwaves = gridDim.x * (blockDim.x / 64);
  const uint32_t C = (uint32_t)min<int64_t>((int64_t)*n_chunks, cmax);
  for (uint32_t c = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); c < C; c += nwaves) {
    const ChunkSpan cs = chunk_span(c, chunk_sb, chunk_base, sb_ranges, S, SX);
    uint32_t mycount = 0;  // lane u < 16 accumulates tile u
    for (int64_t base = cs.begin; base < cs.end; base += 64) {
      const int64_t q = base + lane;
      const bool act = q < cs.end;
      const Packed g = unpack(act ? pval[q] : 0ull);
      const StepMasks m = step_masks(act, g, cs.sx, cs.sy);
      mycount += (uint32_t)__popcll(lane_tile_mask(m, lane));
    }
    if (lane < 16) {
      cnt[(int64_t)c * 16 + lane] = mycount;
      const int t = tile_of(cs.sx, cs.sy, lane, TX, TY);
      if (t >= 0 && mycount) atomicAdd(&tot[t], mycount);
    }
  }
}

// 4b + 5. One block: ranges = exclusive scan of the tile totals, and the stats.
__global__ __launch_bounds__(kBig) void tile_scan_stats_kernel(const uint32_t* __restrict__ tot, int T,
                                                               const uint32_t* __restrict__ blkstat, int nblk,
                                                               int64_t cap, int32_t* __restrict__ ranges,
                                                               int32_t* __restrict__ stats) {
  __shared__ uint32_t carry;
  __shared__ int64_t red[7][kBig / 64];
  if (threadIdx.x == 0) carry = 0;
  int64_t acc[7] = {0, 0, 0, 0, 0, 0, 0};  // max, ovf tiles, ovf inter, trunc tiles, trunc inter, cap, neg
  __syncthreads();
  for (int t0 = 0; t0 < T; t0 += kBig) {
    const int t = t0 + threadIdx.x;
    const uint32_t c = t < T ? tot[t] : 0u;
    uint32_t sum;
    const uint32_t ex = block_excl_scan<kBig>(c, &sum);
    if (t < T) ranges[t] = (int32_t)(carry + ex);
    acc[0] = acc[0] > (int64_t)c ? acc[0] : (int64_t)c;
    acc[1] += c > (uint32_t)kBlock;
    acc[2] += c > (uint32_t)kBlock ? c - kBlock : 0;
    acc[3] += c > (uint32_t)kMaxTileEntries;
    acc[4] += c > (uint32_t)kMaxTileEntries ? c - kMaxTileEntries : 0;
    __syncthreads();
    if (threadIdx.x == 0) carry += sum;
    __syncthreads();
  }
  for (int b = threadIdx.x; b < nblk; b += kBig) {
    acc[5] += blkstat[2 * b];
    acc[6] += blkstat[2 * b + 1];
  }
  // reduce the 7 accumulators over the block
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 7; ++k) {
    int64_t v = acc[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const int64_t w = __shfl_xor(v, o, 64);
      v = k == 0 ? (v > w ? v : w) : v + w;
    }
    if (lane == 0) red[k][wid] = v;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t r[7] = {0, 0, 0, 0, 0, 0, 0};
    for (int w = 0; w < kBig / 64; ++w)
      for (int k = 0; k < 7; ++k) r[k] = k == 0 ? (r[0] > red[0][w] ? r[0] : red[0][w]) : r[k] + red[k][w];
    const int64_t m = carry;
    ranges[T] = (int32_t)m;
    for (int k = 0; k < GS_NUM_STATS; ++k) stats[k] = 0;
    stats[GS_STAT_N_INTERACTIONS] = (int32_t)m;
    stats[GS_STAT_MAX_PER_TILE] = (int32_t)r[0];
    stats[GS_STAT_OVERFLOW_TILES] = (int32_t)r[1];
    stats[GS_STAT_OVERFLOW_INTERACTIONS] = (int32_t)r[2];
    stats[GS_STAT_TRUNCATED_TILES] = (int32_t)r[3];
    stats[GS_STAT_TRUNCATED_INTERACTIONS] = (int32_t)r[4];
    stats[GS_STAT_RADIUS_CAP_VIOLATIONS] = (int32_t)r[5];
    stats[GS_STAT_NEGATIVE_DEPTH] = (int32_t)r[6];
    stats[GS_STAT_CAPACITY_EXCEEDED] = m > cap ? 1 : 0;
  }
}

// 4c. write every entry: tile t's entries from chunk c start at ranges[t] plus the
// counts of the superblock's earlier chunks; within a step, lane L's entry in tile u
// is preceded by popcount(mask_u & lanes-below-L).
__global__ __launch_bounds__(256) void tile_write_kernel(const uint32_t* __restrict__ n_chunks, int64_t cmax,
                                                         const uint32_t* __restrict__ chunk_sb,
                                                         const uint32_t* __restrict__ chunk_base,
                                                         const int32_t* __restrict__ sb_ranges, int S,
                                                         const uint64_t* __restrict__ pval, uint32_t n_gauss, int SX,
                                                         int TX, int TY, const uint32_t* __restrict__ cnt,
                                                         const int32_t* __restrict__ ranges, int64_t cap,
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
    if (lane < 16) {
      const int t = tile_of(cs.sx, cs.sy, lane, TX, TY);
      uint32_t b = t >= 0 ? (uint32_t)ranges[t] : 0u;
      for (uint32_t c2 = cs.first; c2 < c; ++c2) b += cnt[(int64_t)c2 * 16 + lane];
      sbase[wid][lane] = b;
    }
    for (int64_t base = cs.begin; base < cs.end; base += 64) {
      const int64_t q = base + lane;
      bool act = q < cs.end;
      const Packed g = unpack(act ? pval[q] : 0ull);
      act = act && g.gid < n_gauss;  // ids are < n by construction
      const StepMasks m = step_masks(act, g, cs.sx, cs.sy);
      const uint64_t mine = lane_tile_mask(m, lane);
      if (lane < 16) smask[wid][lane] = mine;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (act) {
        const int ux0 = max(g.x0, cs.sx * kSB), ux1 = min(g.x0 + g.w, cs.sx * kSB + kSB);
        const int uy0 = max(g.y0, cs.sy * kSB), uy1 = min(g.y0 + g.h, cs.sy * kSB + kSB);
        for (int ty = uy0; ty < uy1; ++ty)
          for (int tx = ux0; tx < ux1; ++tx) {
            const int u = (ty - cs.sy * kSB) * kSB + (tx - cs.sx * kSB);
            const int64_t dst = (int64_t)sbase[wid][u] + __popcll(smask[wid][u] & lt);
            if (dst < cap) {
              out_gid[dst] = (int32_t)g.gid;
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
  size_t o_dkey, o_word, o_ka, o_wa, o_kb, o_wb, o_off, o_part, o_table, o_dtot, o_scal, o_pk0, o_pv0, o_pk1,
      o_pv1, o_sbr, o_cbase, o_csb, o_cnt, o_tot, o_blk, total;
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
  P.G_d = (int)((nn + kPrepSpan - 1) / kPrepSpan);
  P.G_p = (int)std::min<int64_t>(8192, std::max<int64_t>(1, (2 * nn + 1023) / 1024));
  const int64_t tbl = (int64_t)kRadixBins * std::max(P.G_d, P.G_p);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  P.o_dkey = take(nn * 4);
  P.o_word = take(nn * 8);
  P.o_ka = take(nn * 4);
  P.o_wa = take(nn * 8);
  P.o_kb = take(nn * 4);
  P.o_wb = take(nn * 8);
  P.o_off = take((nn + 1) * 4);
  P.o_part = take((size_t)div_up(nn, kScanTile) * 4 + 64);
  P.o_table = take((size_t)tbl * 4);
  P.o_dtot = take(kRadixBins * 4);
  P.o_scal = take(256);  // device scalars: [0] pairs, [1] chunks
  P.o_pk0 = take((size_t)P.pcap * 4);
  P.o_pv0 = take((size_t)P.pcap * 8);
  P.o_pk1 = take((size_t)P.pcap * 4);
  P.o_pv1 = take((size_t)P.pcap * 8);
  P.o_sbr = take(((size_t)P.S + 1) * 4);
  P.o_cbase = take(((size_t)P.S + 1) * 4);
  P.o_csb = take((size_t)P.cmax * 4);
  P.o_cnt = take((size_t)P.cmax * 16 * 4);
  P.o_tot = take((size_t)P.T * 4);
  P.o_blk = take((size_t)P.G_d * 2 * 4);
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
  hipLaunchKernelGGL(scan_down_kernel<Load>, dim3(nb), dim3(kScanBlock), 0, s, load, n, partial, out,
                     (const uint32_t*)total);
  GS_LAUNCH_CHECK("scan_down_kernel");
  return GS_OK;
}

// One stable radix pass: keys_in/vals_in -> keys_out/vals_out on digit `shift`.
// The upsweep is skipped when the table was already filled (first depth pass).
int radix_pass(hipStream_t s, bool upsweep, const uint32_t* kin, const uint64_t* vin, uint32_t* kout, uint64_t* vout,
               const uint32_t* n_dev, int64_t n_static, int64_t cap, int shift, int G, int fixed_chunk,
               uint32_t* table, uint32_t* dtot) {
  if (upsweep) {
    hipLaunchKernelGGL(radix_upsweep_kernel, dim3(G), dim3(64), 0, s, kin, n_dev, n_static, cap, shift, G,
                       fixed_chunk, table);
    GS_LAUNCH_CHECK("radix_upsweep_kernel");
  }
  hipLaunchKernelGGL(radix_spine_kernel, dim3(kRadixBins), dim3(kScanBlock), 0, s, table, G, dtot);
  GS_LAUNCH_CHECK("radix_spine_kernel");
  hipLaunchKernelGGL(radix_downsweep_kernel, dim3(G), dim3(64), 0, s, kin, vin, n_dev, n_static, cap, shift, G,
                     fixed_chunk, table, dtot, kout, vout);
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
  GS_REQUIRE(width > 0 && height > 0 && width <= 4096 * kTile && height <= 4096 * kTile,
             "gs_bin: bad image size %dx%d (each side at most 65536)", width, height);
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
  uint64_t* word = (uint64_t*)(ws + P.o_word);
  uint32_t* ka = (uint32_t*)(ws + P.o_ka);
  uint64_t* wa = (uint64_t*)(ws + P.o_wa);
  uint32_t* kb = (uint32_t*)(ws + P.o_kb);
  uint64_t* wb = (uint64_t*)(ws + P.o_wb);
  uint32_t* off = (uint32_t*)(ws + P.o_off);
  uint32_t* part = (uint32_t*)(ws + P.o_part);
  uint32_t* table = (uint32_t*)(ws + P.o_table);
  uint32_t* dtot = (uint32_t*)(ws + P.o_dtot);
  uint32_t* scal = (uint32_t*)(ws + P.o_scal);
  uint32_t* pk0 = (uint32_t*)(ws + P.o_pk0);
  uint64_t* pv0 = (uint64_t*)(ws + P.o_pv0);
  uint32_t* pk1 = (uint32_t*)(ws + P.o_pk1);
  uint64_t* pv1 = (uint64_t*)(ws + P.o_pv1);
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
  // 1. prep (+ histogram of the first depth digit)
  hipLaunchKernelGGL(bin_prep_kernel, dim3(P.G_d), dim3(kPrepBlock), 0, s, n, means2d, radii, valid, depths, width,
                     height, P.G_d, dkey, word, table, blk);
  GS_LAUNCH_CHECK("bin_prep_kernel");
  // 2. stable depth sort of the packed words (13-bit bucket: 7 + 6 bits)
  int rc = radix_pass(s, false, dkey, word, kb, wb, nullptr, n, n, 0, P.G_d, kPrepSpan, table, dtot);
  if (rc != GS_OK) return rc;
  rc = radix_pass(s, true, kb, wb, ka, wa, nullptr, n, n, kRadixBits, P.G_d, kPrepSpan, table, dtot);
  if (rc != GS_OK) return rc;
  const uint64_t* sorted_word = wa;
  // 3. superblock pairs in depth order, stably sorted by superblock
  rc = run_scan(s, LoadSortedSB{sorted_word}, n, part, off, n_pairs);
  if (rc != GS_OK) return rc;
  hipLaunchKernelGGL(sb_pairs_kernel, dim3(div_up(n, 256)), dim3(256), 0, s, n, sorted_word, off, P.pcap, P.SX, pk0,
                     pv0);
  GS_LAUNCH_CHECK("sb_pairs_kernel");
  uint32_t* sbkey = pk0;
  uint64_t* sbval = pv0;
  if (P.sb_passes >= 1) {
    rc = radix_pass(s, true, pk0, pv0, pk1, pv1, n_pairs, 0, P.pcap, 0, P.G_p, 0, table, dtot);
    if (rc != GS_OK) return rc;
    sbkey = pk1;
    sbval = pv1;
  }
  if (P.sb_passes == 2) {
    rc = radix_pass(s, true, pk1, pv1, pk0, pv0, n_pairs, 0, P.pcap, kRadixBits, P.G_p, 0, table, dtot);
    if (rc != GS_OK) return rc;
    sbkey = pk0;
    sbval = pv0;
  }
  hipLaunchKernelGGL(ranges_kernel, dim3(std::min(2048, div_up(P.pcap + 1, 256))), dim3(256), 0, s, sbkey, n_pairs,
                     P.pcap, P.S, sbr);
  GS_LAUNCH_CHECK("ranges_kernel");
  // 4. tile pass
  hipLaunchKernelGGL(chunks_kernel, dim3(1), dim3(kBig), 0, s, P.S, sbr, P.cmax, cbase, csb, n_chunks, P.T, tot);
  GS_LAUNCH_CHECK("chunks_kernel");
  const int pass_blocks = 2048;
  hipLaunchKernelGGL(tile_count_kernel, dim3(pass_blocks), dim3(256), 0, s, n_chunks, P.cmax, csb, cbase, sbr, P.S,
                     sbval, P.SX, P.TX, P.TY, cnt, tot);
  GS_LAUNCH_CHECK("tile_count_kernel");
  hipLaunchKernelGGL(tile_scan_stats_kernel, dim3(1), dim3(kBig), 0, s, tot, P.T, blk, P.G_d, P.cap, ranges, stats);
  GS_LAUNCH_CHECK("tile_scan_stats_kernel");
  hipLaunchKernelGGL(tile_write_kernel, dim3(pass_blocks), dim3(256), 0, s, n_chunks, P.cmax, csb, cbase, sbr, P.S,
                     sbval, (uint32_t)n, P.SX, P.TX, P.TY, cnt, ranges, P.cap, sorted_gids, sorted_tiles);
  GS_LAUNCH_CHECK("tile_write_kernel");
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
