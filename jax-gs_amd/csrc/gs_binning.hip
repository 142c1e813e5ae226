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
//   3. superblocks     a superblock is 8x8 tiles; a Gaussian (at most 16 tiles a side)
//                      meets at most 3x3 of them.  Its (superblock, word) pairs are
//                      generated on the fly from the depth-sorted words and counting-
//                      sorted by superblock in one 8-bit radix pass (two when the image
//                      has more than 256 superblocks) -> per superblock the list of
//                      Gaussians touching it, in (bucket, id) order.  A wave lists the
//                      pairs of its 64 Gaussians in LDS in Gaussian order and ranks
//                      the list 64 pairs at a time; a Gaussian has one pair per
//                      superblock at most, so each superblock's pairs keep Gaussian
//                      order.
//   4. tile pass       a superblock's list is cut into chunks of 256 Gaussians; a wave
//                      takes a chunk 64 Gaussians at a time and forms 8 column and 8
//                      row lane masks with ballots; lane u owns tile u of the
//                      superblock and its mask (column & row) says which Gaussians of
//                      the step hit it.  A counting sweep gives per (chunk, tile) counts,
//                      a two-level scan (segments of 16 chunks, then each superblock's
//                      segments) turns them into chunk offsets and tile totals, one
//                      scan gives the tile ranges, and a writing
//                      sweep stores, tile by tile, the ids of the lanes in the tile's
//                      mask at range + counts of earlier chunks + popcount(mask &
//                      lanes-below): stable by construction, one contiguous run per
//                      store instruction.
//   5. stats           the renderer's health extras, computed with the range scan.
//
// Radix passes use one wave per workgroup over a contiguous range (in-wave rank with
// ballot "match any"), a per-digit spine scan across workgroups, and no
// inter-workgroup waiting.  There are no same-address global atomics.
#include "gs_bins.h"
#include "gs_common.h"

#include <algorithm>
#include <mutex>

namespace gs {
namespace {

constexpr int kScanBlock = 256;
constexpr int kSBSpan = 3;                        // superblocks a Gaussian meets per axis
constexpr int kChunk = 256;                       // Gaussians per chunk of the tile pass
constexpr int kSeg = 16;                          // chunks per segment of the chunk-offset scan
constexpr int kPrepBlock = 256;
constexpr int kPrepPer = 4;                       // Gaussians per bin_prep thread
constexpr int kSpan = kPrepBlock * kPrepPer;      // Gaussians per depth-sort workgroup
constexpr int kPairSpan = 256;                    // Gaussians per superblock-sort workgroup
constexpr int kBig = 1024;                        // single-block kernels
constexpr int kDepthRB = 7;                       // depth buckets: two 7-bit digits
constexpr int kPairRB = 8;                        // superblock ids: 8-bit digits
constexpr int kBlkStats = 3;  // per bin_prep block: cap violations, negative depths, their entries

__device__ inline uint64_t lanemask_lt() {
  const unsigned lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Superblock rectangle [sx0, sx1] x [sy0, sy1] of a Gaussian (empty when w == 0).
struct SBRect {
  int sx0, sx1, sy0, sy1;
  bool has;
};
__device__ inline SBRect sb_rect(const Packed& p) {
  SBRect r;
  r.has = p.w > 0;
  r.sx0 = p.x0 / kSB;
  r.sx1 = (p.x0 + p.w - 1) / kSB;
  r.sy0 = p.y0 / kSB;
  r.sy1 = (p.y0 + p.h - 1) / kSB;
  return r;
}

// Lanes (among `act` lanes) whose value d (RB bits) equals this lane's.
template <int RB>
__device__ inline uint64_t match_any(uint32_t d, bool act) {
  uint64_t m = __ballot(act);
#pragma unroll
  for (int bb = 0; bb < RB; ++bb) {
    const bool bit = (d >> bb) & 1u;
    const uint64_t bm = __ballot(bit);
    m &= bit ? bm : ~bm;
  }
  return m;
}

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

// rasterizer.py:36-51 for one Gaussian: the tile rectangle of its box clipped to the
// image (floor(x / 16) of clipped coordinates; NaN, only for invalid Gaussians,
// converts to 0 as XLA's does), the strict on-screen test, and v, whether its slots
// hold entries; count = the number of entries (slots of the 16 x 16 offset grid inside
// the rectangle, rasterizer.py:56-69).
struct TileRect {
  int tminx, tminy, spanx, spany;
  bool proj_valid, on_screen, v;
  __device__ int count() const { return v ? (spanx < kOffset ? spanx : kOffset) * (spany < kOffset ? spany : kOffset) : 0; }
};
__device__ inline TileRect tile_rect(float mx, float my, float rr, bool proj_valid, int W, int H) {
  TileRect t;
  const float wm1 = (float)(W - 1), hm1 = (float)(H - 1);
  const float minx = jmin(jmax(mx - rr, 0.0f), wm1);
  const float maxx = jmin(jmax(mx + rr, 0.0f), wm1);
  const float miny = jmin(jmax(my - rr, 0.0f), hm1);
  const float maxy = jmin(jmax(my + rr, 0.0f), hm1);
  t.tminx = (int)floorf(minx / 16.0f);
  t.tminy = (int)floorf(miny / 16.0f);
  const int tmaxx = (int)floorf(maxx / 16.0f), tmaxy = (int)floorf(maxy / 16.0f);
  t.on_screen = (mx + rr > 0.0f) && (mx - rr < (float)W) && (my + rr > 0.0f) && (my - rr < (float)H);
  t.proj_valid = proj_valid;
  t.v = proj_valid && t.on_screen && (tmaxx >= t.tminx) && (tmaxy >= t.tminy);
  t.spanx = tmaxx - t.tminx + 1;
  t.spany = tmaxy - t.tminy + 1;
  return t;
}

// ---------------------------------------------------------------------------------
// 1. per-Gaussian rectangle and depth bucket (rasterizer.py:36-51, 84-94;
//    renderer.py:63-75 for the radius-cap statistic).  Block b handles Gaussians
//    [b*1024, b*1024+1024), the range of depth-sort workgroup b, and writes that
//    workgroup's histogram of the first radix digit.
__global__ __launch_bounds__(kPrepBlock) void bin_prep_kernel(int64_t n, const float* __restrict__ means2d,
                                                              const float* __restrict__ radii,
                                                              const uint8_t* __restrict__ valid,
                                                              const float* __restrict__ depths, int W, int H, int G,
                                                              uint32_t* __restrict__ dkey, uint64_t* __restrict__ word,
                                                              uint32_t* __restrict__ table,
                                                              uint32_t* __restrict__ blkstat,
                                                              uint4* __restrict__ zero_buf, int64_t n_zero4) {
  constexpr int NB = 1 << kDepthRB;
  {
    // the tile pass's segment totals, accumulated with atomics later: cleared here
    const int64_t per = (n_zero4 + gridDim.x - 1) / gridDim.x;
    const int64_t z0 = per * blockIdx.x, z1 = z0 + per < n_zero4 ? z0 + per : n_zero4;
    for (int64_t z = z0 + threadIdx.x; z < z1; z += kPrepBlock) zero_buf[z] = make_uint4(0u, 0u, 0u, 0u);
  }
  __shared__ uint32_t hist[NB];
  __shared__ uint32_t wcnt[kBlkStats][kPrepBlock / 64];
  for (int d = threadIdx.x; d < NB; d += kPrepBlock) hist[d] = 0;
  __syncthreads();
  uint32_t capc = 0, negc = 0, neg_entries = 0;
  for (int r = 0; r < kPrepPer; ++r) {
    const int64_t i = (int64_t)blockIdx.x * kSpan + r * kPrepBlock + threadIdx.x;
    bool cap_violation = false, negative = false;
    if (i < n) {
      const TileRect t = tile_rect(means2d[2 * i], means2d[2 * i + 1], radii[i], valid[i] != 0, W, H);
      cap_violation = t.proj_valid && t.on_screen && (t.spanx > kOffset || t.spany > kOffset);
      const uint32_t zb = float_to_bits(depths[i]);
      negative = (zb >> 31) != 0;
      // A depth with its sign bit set makes every key of the Gaussian negative, so its
      // valid slots sort in front with tile -1 (rasterizer.py:98-104): they count as
      // interactions but are no tile's entries.  (project_gaussians never marks such a
      // Gaussian valid; get_tile_interactions' caller may.)
      const bool e = t.v && !negative;
      if (t.v && negative) neg_entries += (uint32_t)t.count();
      uint32_t key = kDepthBinEmpty;
      int w = 0, h = 0;
      if (e) {
        w = t.spanx < kOffset ? t.spanx : kOffset;
        h = t.spany < kOffset ? t.spany : kOffset;
        key = depth_key(zb);
      }
      dkey[i] = key;
      word[i] = pack((uint32_t)i, e ? t.tminx : 0, e ? t.tminy : 0, w, h);
      // Gaussians that meet no tile are dropped by the first radix pass: not counted
      if (e) atomicAdd(&hist[key & (NB - 1)], 1u);
    }
    capc += (uint32_t)__popcll(__ballot(cap_violation));
    negc += (uint32_t)__popcll(__ballot(negative));
  }
  // entries of negative-depth Gaussians: a wave sum (at most 256 per Gaussian)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) neg_entries += __shfl_xor(neg_entries, o, 64);
  if ((threadIdx.x & 63) == 0) {
    wcnt[0][threadIdx.x >> 6] = capc;
    wcnt[1][threadIdx.x >> 6] = negc;
    wcnt[2][threadIdx.x >> 6] = neg_entries;
  }
  __syncthreads();
  if (threadIdx.x < kBlkStats) {
    uint32_t s = 0;
    for (int k = 0; k < kPrepBlock / 64; ++k) s += wcnt[threadIdx.x][k];
    blkstat[kBlkStats * (int64_t)blockIdx.x + threadIdx.x] = s;
  }
  for (int d = threadIdx.x; d < NB; d += kPrepBlock) table[(int64_t)d * G + blockIdx.x] = hist[d];
}

// ---------------------------------------------------------------------------------
// Stable LSD radix pass on an RB-bit digit at `shift`, keys u32 + values u64.
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

template <int RB>
__global__ __launch_bounds__(64) void radix_upsweep_kernel(const uint32_t* __restrict__ keys,
                                                           const uint32_t* __restrict__ n_dev,
                                                           int64_t n_static, int64_t cap, int shift, int G,
                                                           int fixed_chunk, uint32_t* __restrict__ table) {
  constexpr int NB = 1 << RB;
  __shared__ uint32_t hist[NB];
  const int lane = threadIdx.x;
  for (int d = lane; d < NB; d += 64) hist[d] = 0;
  __syncthreads();
  int64_t begin, end;
  pass_range(n_dev, n_static, cap, G, fixed_chunk, begin, end);
  for (int64_t i = begin + lane; i < end; i += 64) atomicAdd(&hist[(keys[i] >> shift) & (NB - 1)], 1u);
  __syncthreads();
  for (int d = lane; d < NB; d += 64) table[(int64_t)d * G + blockIdx.x] = hist[d];
}

// One block per digit: exclusive scan of that digit's row of the table (over the G
// workgroups) in place, and the digit's total.  The row moves through LDS in pieces of up to
// kSpineMax entries with coalesced loads and stores (a running carry joins the pieces); each
// thread scans a contiguous run of a piece.  The LDS copy is skewed by one word per 32
// (entry k at k + k / 32): the runs start `per` words apart, which unskewed put a wave's
// reads on two banks when per is 16 (the superblock pass at 1M Gaussians: 3907 workgroups).
// Rows longer than one piece (the superblock pass above 2M Gaussians: 11,719 workgroups at
// 3M) were scanned from global memory by the threads' runs, uncoalesced: 33 us at 3M.
constexpr int kSpineMax = 8192;
constexpr int kSpineBatch = 8;  // global loads (stores) per thread in flight at once
static_assert(kSpineMax % (kSpineBatch * kScanBlock) == 0, "batches tile a piece");
__device__ inline int spine_at(int k) { return k + (k >> 5); }
__global__ __launch_bounds__(kScanBlock) void radix_spine_kernel(uint32_t* __restrict__ table, int G,
                                                                 uint32_t* __restrict__ digit_tot) {
  __shared__ uint32_t row_s[kSpineMax + kSpineMax / 32];
  const int d = blockIdx.x;
  uint32_t* row = table + (int64_t)d * G;
  uint32_t carry = 0;
  for (int c0 = 0; c0 < G; c0 += kSpineMax) {
    const int len = G - c0 < kSpineMax ? G - c0 : kSpineMax;
    // The piece into LDS, kSpineBatch loads per thread issued before any of them is stored
    // (one load waited for at a time made each thread a chain of round trips: 23 us for the
    // 11,719-entry rows of 3M Gaussians).  k0 steps by kSpineBatch * kScanBlock, which divides
    // kSpineMax, so every k below is inside the LDS array.
    for (int k0 = 0; k0 < len; k0 += kSpineBatch * kScanBlock) {
      uint32_t v[kSpineBatch];
#pragma unroll
      for (int u = 0; u < kSpineBatch; ++u) {
        const int k = k0 + u * kScanBlock + threadIdx.x;
        v[u] = k < len ? row[c0 + k] : 0u;
      }
#pragma unroll
      for (int u = 0; u < kSpineBatch; ++u) {
        const int k = k0 + u * kScanBlock + threadIdx.x;
        if (k < len) row_s[spine_at(k)] = v[u];
      }
    }
    __syncthreads();
    // each thread's run, branch-free (per * kScanBlock <= kSpineMax: slots past len are inside
    // the array; they are read as 0 and what is written there is never stored)
    const int per = (len + kScanBlock - 1) / kScanBlock;
    const int b0 = threadIdx.x * per;
    uint32_t s = 0, tot;
#pragma unroll 8
    for (int k = 0; k < per; ++k) {
      const uint32_t x = row_s[spine_at(b0 + k)];
      s += b0 + k < len ? x : 0u;
    }
    uint32_t run = carry + block_excl_scan<kScanBlock>(s, &tot);
#pragma unroll 8
    for (int k = 0; k < per; ++k) {
      const uint32_t x = row_s[spine_at(b0 + k)];
      row_s[spine_at(b0 + k)] = run;
      run += x;
    }
    __syncthreads();
    for (int k0 = 0; k0 < len; k0 += kSpineBatch * kScanBlock) {
      uint32_t v[kSpineBatch];
#pragma unroll
      for (int u = 0; u < kSpineBatch; ++u) v[u] = row_s[spine_at(k0 + u * kScanBlock + threadIdx.x)];
#pragma unroll
      for (int u = 0; u < kSpineBatch; ++u) {
        const int k = k0 + u * kScanBlock + threadIdx.x;
        if (k < len) row[c0 + k] = v[u];
      }
    }
    carry += tot;
    __syncthreads();  // the piece's stores read row_s before the next piece overwrites it
  }
  if (threadIdx.x == 0) digit_tot[d] = carry;
}

// Per-lane digit counters of workgroup g: base of each digit (exclusive scan of the
// digit totals) plus the workgroup's offset within the digit.  Returns the total.
template <int RB>
__device__ inline uint32_t init_digit_counters(uint32_t* cnt, const uint32_t* __restrict__ table,
                                               const uint32_t* __restrict__ digit_tot, int G, int g, int lane) {
  constexpr int DPL = (1 << RB) / 64;  // digits per lane
  uint32_t a[DPL], sum = 0;
#pragma unroll
  for (int k = 0; k < DPL; ++k) {
    a[k] = digit_tot[DPL * lane + k];
    sum += a[k];
  }
  const uint32_t inc = wave_incl_scan(sum);
  uint32_t base = inc - sum;
#pragma unroll
  for (int k = 0; k < DPL; ++k) {
    cnt[DPL * lane + k] = base + table[(int64_t)(DPL * lane + k) * G + g];
    base += a[k];
  }
  return __shfl(inc, 63, 64);
}

constexpr int kUnroll = 4;

// drop_empty: keys equal to kDepthBinEmpty (Gaussians meeting no tile, left out of the
// histogram) are not written, so the output holds only the others, still stable; the
// pass's output count goes to *n_kept (when given).
template <int RB>
__global__ __launch_bounds__(64) void radix_downsweep_kernel(
    const uint32_t* __restrict__ keys_in, const uint64_t* __restrict__ vals_in, const uint32_t* __restrict__ n_dev,
    int64_t n_static, int64_t cap, int shift, int G, int fixed_chunk, const uint32_t* __restrict__ table,
    const uint32_t* __restrict__ digit_tot, uint32_t* __restrict__ keys_out, uint64_t* __restrict__ vals_out,
    bool drop_empty, uint32_t* __restrict__ n_kept) {
  constexpr int NB = 1 << RB;
  __shared__ uint32_t cnt[NB];
  const int lane = threadIdx.x;
  const uint32_t total = init_digit_counters<RB>(cnt, table, digit_tot, G, blockIdx.x, lane);
  if (n_kept != nullptr && blockIdx.x == 0 && lane == 0) *n_kept = total;
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
      const bool a = i < end && !(drop_empty && k[u] == (uint32_t)kDepthBinEmpty);
      const uint32_t d = (k[u] >> shift) & (NB - 1);
      const uint64_t m = match_any<RB>(d, a);
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
// 3. Superblock pairs, generated from the depth-sorted words.  Workgroup g covers
// Gaussians [g*256, (g+1)*256) (depth-sorted positions); the pass sorts on the low
// 8 bits of the superblock id.
__global__ __launch_bounds__(256) void pair_upsweep_kernel(const uint64_t* __restrict__ words, int64_t n_static,
                                                           const uint32_t* __restrict__ n_dev, int SX, int G,
                                                           uint32_t* __restrict__ table) {
  const int64_t n = n_static < (int64_t)*n_dev ? n_static : (int64_t)*n_dev;  // Gaussians with tiles
  constexpr int NB = 1 << kPairRB;
  // column g of the table: workgroups of one XCD (b mod 8) take a contiguous run of
  // columns, so each row's cache lines are written by one L2
  const int per = (G + 7) >> 3;
  const int g = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (g >= G) return;
  __shared__ uint32_t hist[NB];
  hist[threadIdx.x] = 0;
  __syncthreads();
  static_assert(kPairSpan == 256, "one Gaussian per thread");
  const int64_t i = (int64_t)g * kPairSpan + threadIdx.x;
  if (i < n) {
    const SBRect b = sb_rect(unpack(words[i]));
    if (b.has)
      for (int sy = b.sy0; sy <= b.sy1; ++sy)
        for (int sx = b.sx0; sx <= b.sx1; ++sx) atomicAdd(&hist[(uint32_t)(sy * SX + sx) & (NB - 1)], 1u);
  }
  __syncthreads();
  table[(int64_t)threadIdx.x * G + g] = hist[threadIdx.x];
}

// The chunk and segment maps of the tile pass (chunks_kernel's outputs) computed inside
// the superblock pass when the pass has one round (S <= 256: a superblock id is its
// digit, so its pair range follows from the digit totals, final before the pass
// starts).  Every workgroup scans the <= 256 totals itself (one wave, four superblocks
// per lane) and fills its own slice of the chunk -> superblock and segment ->
// superblock maps; workgroup 0 writes the bases and counts.  No workgroup waits for
// another.
struct ChunkMapArgs {
  int S;
  int64_t cmax, gmax;
  int32_t* sb_ranges;
  uint32_t *chunk_base, *chunk_sb, *n_chunks, *seg_base, *n_segs;
};

__device__ inline void chunk_maps_from_digits(const ChunkMapArgs& A, const uint32_t* __restrict__ digit_tot,
                                              uint32_t* cb, int lane) {
  constexpr int PER = 256 / 64;  // superblocks per lane
  uint32_t cnt[PER], nc[PER], ng[PER], sum_p = 0, sum_c = 0, sum_g = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int sb = PER * lane + k;
    cnt[k] = sb < A.S ? digit_tot[sb] : 0u;
    nc[k] = (cnt[k] + kChunk - 1) / kChunk;
    ng[k] = (nc[k] + kSeg - 1) / kSeg;
    sum_p += cnt[k];
    sum_c += nc[k];
    sum_g += ng[k];
  }
  const uint32_t ip = wave_incl_scan(sum_p), ic = wave_incl_scan(sum_c), ig = wave_incl_scan(sum_g);
  uint32_t p = ip - sum_p, c = ic - sum_c, g = ig - sum_g;
  const bool w0 = blockIdx.x == 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int sb = PER * lane + k;
    if (sb < A.S) {
      cb[sb] = c;
      if (w0) {
        A.sb_ranges[sb] = (int32_t)p;
        A.chunk_base[sb] = c;
        A.seg_base[sb] = g;
      }
    }
    p += cnt[k];
    c += nc[k];
    g += ng[k];
  }
  const uint32_t tp = (uint32_t)__shfl(ip, 63, 64), tc = (uint32_t)__shfl(ic, 63, 64),
                 tg = (uint32_t)__shfl(ig, 63, 64);
  if (lane == 0) {
    cb[A.S] = tc;
    if (w0) {
      A.sb_ranges[A.S] = (int32_t)tp;
      A.chunk_base[A.S] = tc;
      A.seg_base[A.S] = tg;
      *A.n_chunks = tc;
      *A.n_segs = tg;
    }
  }
  __syncthreads();
  // this workgroup's slice of the chunk map: chunk j belongs to the last superblock
  // whose base is <= j
  const uint32_t G = gridDim.x;
  const uint32_t nch = (int64_t)tc < A.cmax ? tc : (uint32_t)A.cmax;
  const uint32_t pc = (nch + G - 1) / G;
  for (uint32_t j = blockIdx.x * pc + lane; j < nch && j < (blockIdx.x + 1) * pc; j += 64) {
    int lo = 0, hi = A.S;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (cb[mid] <= j) lo = mid; else hi = mid;
    }
    A.chunk_sb[j] = (uint32_t)lo;
  }
}

// Each round of 64 Gaussians lists its (superblock, lane) pairs in LDS in lane order
// (a wave prefix sum of the pair counts gives each Gaussian its place) and ranks the
// list 64 pairs at a time.  A Gaussian has at most one pair per superblock, so the
// pairs of any one superblock stay in Gaussian order: the pass is stable.
template <bool WITH_KEYS>
__global__ __launch_bounds__(64) void pair_downsweep_kernel(const uint64_t* __restrict__ words, int64_t n_static,
                                                            const uint32_t* __restrict__ n_dev, int SX,
                                                            int G, const uint32_t* __restrict__ table,
                                                            const uint32_t* __restrict__ digit_tot,
                                                            uint32_t* __restrict__ keys_out,
                                                            uint64_t* __restrict__ vals_out,
                                                            uint32_t* __restrict__ n_pairs, ChunkMapArgs maps) {
  constexpr int NB = 1 << kPairRB;
  __shared__ uint32_t cnt[NB];
  __shared__ uint32_t mcb[NB + 1];
  __shared__ uint32_t list[64 * kSBSpan * kSBSpan];  // (superblock << 6) | lane
  __shared__ uint64_t wl[64];
  const int lane = threadIdx.x;
  const uint32_t total = init_digit_counters<kPairRB>(cnt, table, digit_tot, G, blockIdx.x, lane);
  if (blockIdx.x == 0 && lane == 0) *n_pairs = total;
  const int64_t n = n_static < (int64_t)*n_dev ? n_static : (int64_t)*n_dev;  // Gaussians with tiles
  if (maps.S > 0) chunk_maps_from_digits(maps, digit_tot, mcb, lane);
  __syncthreads();
  const int64_t begin = (int64_t)blockIdx.x * kPairSpan;
  const int64_t end = begin + kPairSpan < n ? begin + kPairSpan : n;
  const uint64_t lt = lanemask_lt();
  for (int64_t base = begin; base < end; base += 64) {
    const int64_t i = base + lane;
    const bool in = i < end;
    const uint64_t wv = in ? words[i] : 0ull;
    const SBRect b = sb_rect(unpack(wv));
    const int nx = (in && b.has) ? b.sx1 - b.sx0 + 1 : 0;
    const int ny = (in && b.has) ? b.sy1 - b.sy0 + 1 : 0;
    const uint32_t c = (uint32_t)(nx * ny);
    const uint32_t inc = wave_incl_scan(c);
    const uint32_t P = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
    uint32_t at = inc - c;
    wl[lane] = wv;
    for (int jy = 0; jy < ny; ++jy)
      for (int jx = 0; jx < nx; ++jx) list[at++] = ((uint32_t)((b.sy0 + jy) * SX + b.sx0 + jx) << 6) | (uint32_t)lane;
    __syncthreads();
    for (uint32_t b0 = 0; b0 < P; b0 += 64) {
      const bool act = b0 + lane < P;
      const uint32_t e = act ? list[b0 + lane] : 0u;
      const uint32_t sb = e >> 6;
      const uint32_t d = sb & (NB - 1);
      const uint64_t m = match_any<kPairRB>(d, act);
      if (act) {
        const uint64_t before = m & lt;
        const uint32_t base_d = cnt[d];
        const uint32_t dst = base_d + (uint32_t)__popcll(before);
        // All lanes have read cnt[] before the group's first lane writes it back:
        // LDS operations of one wave execute in program order.
        if (before == 0) cnt[d] = base_d + (uint32_t)__popcll(m);
        if (dst < total) {  // always true for a consistent table
          vals_out[dst] = wl[e & 63];
          if (WITH_KEYS) keys_out[dst] = sb;
        }
      }
    }
    __syncthreads();  // the list and words are rewritten by the next round
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

// One block, for images whose superblock sort takes two passes (more than 256
// superblocks; with one pass the superblock pass builds these maps itself): chunk count
// per superblock (from the superblock ranges) -> exclusive scan -> chunk_base[S+1] and
// the chunk -> superblock map; likewise the superblock's segments (runs of kSeg chunks,
// the unit of the chunk-offset scan): seg_base[S+1] and the segment -> superblock map.
__global__ __launch_bounds__(kBig) void chunks_kernel(int S, const int32_t* __restrict__ sb_ranges, int64_t cmax,
                                                      uint32_t* __restrict__ chunk_base,
                                                      uint32_t* __restrict__ chunk_sb, uint32_t* __restrict__ n_chunks,
                                                      int64_t gmax, uint32_t* __restrict__ seg_base,
                                                      uint32_t* __restrict__ n_segs) {
  __shared__ uint32_t cb[kBig + 1];  // chunk bases, when S <= kBig
  __shared__ uint32_t carry_c, carry_g;
  if (threadIdx.x == 0) {
    carry_c = 0;
    carry_g = 0;
  }
  __syncthreads();
  for (int s0 = 0; s0 < S; s0 += kBig) {
    const int sb = s0 + threadIdx.x;
    uint32_t lo = 0, hi = 0;
    if (sb < S) {
      lo = (uint32_t)sb_ranges[sb];
      hi = (uint32_t)sb_ranges[sb + 1];
    }
    const uint32_t nc = sb < S ? (hi - lo + kChunk - 1) / kChunk : 0u;
    const uint32_t ng = (nc + kSeg - 1) / kSeg;
    uint32_t sum_c, sum_g;
    const uint32_t c0 = carry_c + block_excl_scan<kBig>(nc, &sum_c);
    const uint32_t g0 = carry_g + block_excl_scan<kBig>(ng, &sum_g);
    if (sb < S) {
      chunk_base[sb] = c0;
      seg_base[sb] = g0;
      if (S <= kBig) {
        cb[sb] = c0;
      } else {
        for (uint32_t c = c0; c < c0 + nc && (int64_t)c < cmax; ++c) chunk_sb[c] = (uint32_t)sb;
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      carry_c += sum_c;
      carry_g += sum_g;
    }
    __syncthreads();
  }
  const uint32_t total = carry_c, total_g = carry_g;
  if (threadIdx.x == 0) {
    chunk_base[S] = total;
    *n_chunks = total;
    seg_base[S] = total_g;
    *n_segs = total_g;
  }
  if (S <= kBig) {
    if (threadIdx.x == 0) {
      cb[S] = total;
    }
    __syncthreads();
    // chunk j belongs to the last superblock whose base is <= j (likewise segments)
    const uint32_t lim = (int64_t)total < cmax ? total : (uint32_t)cmax;
    for (uint32_t j = threadIdx.x; j < lim; j += kBig) {
      int lo = 0, hi = S;  // invariant: cb[lo] <= j < cb[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cb[mid] <= j) lo = mid; else hi = mid;
      }
      chunk_sb[j] = (uint32_t)lo;
    }
  }
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

// Lane u owns tile u of superblock (sx, sy): column u % 8, row u / 8.  Returns the
// lanes (Gaussians of the step) whose rectangle contains that tile: 8 column and 8
// row ballots, and each lane picks its column's and row's mask.
__device__ inline uint64_t tile_lane_mask(bool act, const Packed& g, int sx, int sy, int lane) {
  uint64_t cm = 0, rm = 0;
  const int ux = lane & 7, uy = lane >> 3;
#pragma unroll
  for (int k = 0; k < kSB; ++k) {
    const int tx = sx * kSB + k, ty = sy * kSB + k;
    const uint64_t c = __ballot(act && g.x0 <= tx && tx < g.x0 + g.w);
    const uint64_t r = __ballot(act && g.y0 <= ty && ty < g.y0 + g.h);
    cm = ux == k ? c : cm;
    rm = uy == k ? r : rm;
  }
  return cm & rm;
}

// tile of lane u of superblock (sx, sy), or -1 outside the image
__device__ inline int tile_of(int sx, int sy, int lane, int TX, int TY) {
  const int tx = sx * kSB + (lane & 7), ty = sy * kSB + (lane >> 3);
  return (tx < TX && ty < TY) ? ty * TX + tx : -1;
}

// 4a. counts per (chunk, tile of its superblock) -> cnt[c*64 + u], and the chunk's
// descriptor (first pair, pair count, superblock column and row) for the write sweep.
// The chunk's 256 words are loaded at once (one memory round trip, not four).
static_assert(kChunk == 4 * 64, "a chunk is four steps of 64 Gaussians");
__global__ __launch_bounds__(256) void tile_count_kernel(const uint32_t* __restrict__ n_chunks, int64_t cmax,
                                                         const uint32_t* __restrict__ chunk_sb,
                                                         const uint32_t* __restrict__ chunk_base,
                                                         const int32_t* __restrict__ sb_ranges, int S,
                                                         const uint64_t* __restrict__ pval, int SX,
                                                         const uint32_t* __restrict__ seg_base,
                                                         uint32_t* __restrict__ cnt, uint4* __restrict__ desc,
                                                         uint32_t* __restrict__ seg_sum,
                                                         uint64_t* __restrict__ masks) {
  const int lane = threadIdx.x & 63;
  const uint32_t nwaves = gridDim.x * (blockDim.x / 64);
  const uint32_t C = (uint32_t)min<int64_t>((int64_t)*n_chunks, cmax);
  for (uint32_t c = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); c < C; c += nwaves) {
    const ChunkSpan cs = chunk_span(c, chunk_sb, chunk_base, sb_ranges, S, SX);
    const int len = (int)(cs.end - cs.begin);
    uint64_t wv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) wv[k] = 64 * k + lane < len ? pval[cs.begin + 64 * k + lane] : 0ull;
    uint32_t mycount = 0;  // lane u counts tile u
    uint64_t mk[4] = {0ull, 0ull, 0ull, 0ull};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (64 * k < len) {
        const bool act = 64 * k + lane < len;
        mk[k] = tile_lane_mask(act, unpack(wv[k]), cs.sx, cs.sy, lane);
        mycount += (uint32_t)__popcll(mk[k]);
      }
    }
    cnt[(int64_t)c * 64 + lane] = mycount;
    if (masks != nullptr) {  // (chunk, tile) -> its four step masks, 32 bytes per lane
      ulonglong2* mp = reinterpret_cast<ulonglong2*>(masks + ((int64_t)c * 64 + lane) * 4);
      mp[0] = make_ulonglong2(mk[0], mk[1]);
      mp[1] = make_ulonglong2(mk[2], mk[3]);
    }
    // the chunk's segment (kSeg consecutive chunks of the superblock) and its place in it
    const uint32_t g = seg_base[cs.s] + (c - cs.first) / kSeg, p = (c - cs.first) % kSeg;
    if (mycount != 0u) atomicAdd(&seg_sum[(int64_t)g * 64 + lane], mycount);
    if (lane == 0)
      desc[c] = make_uint4((uint32_t)cs.begin, (uint32_t)len | (p << 16), (uint32_t)cs.sx | ((uint32_t)cs.sy << 16),
                           g);
  }
}

// 4c + 5. One block: ranges = exclusive scan of the tile totals, and the stats.  Rounds
// of 8192 tiles: coalesced loads into LDS, each thread scans 8 consecutive tiles from
// LDS (row stride 9: no bank conflicts), a block scan, prefixes back through LDS and
// coalesced stores.
__global__ __launch_bounds__(kBig) void tile_scan_stats_kernel(const uint32_t* __restrict__ tot, int T,
                                                               const uint32_t* __restrict__ blkstat, int nblk,
                                                               int64_t cap, int64_t n_gauss,
                                                               int32_t* __restrict__ ranges,
                                                               int32_t* __restrict__ stats, bool deferred,
                                                               uint32_t* __restrict__ ticket) {
  constexpr int kPer = 8, kRound = kBig * kPer;
  __shared__ uint32_t stage[kBig * (kPer + 1)];
  __shared__ int64_t red[9][kBig / 64];
  const int tid = threadIdx.x;
  if (tid == 0) *ticket = 0u;  // the write sweep's count of finished workgroups
  // max, ovf tiles, ovf inter, trunc tiles, trunc inter, cap, neg, negative-depth entries,
  // last 512-entry chunk start over the tiles (-1: no entries)
  int64_t acc[9] = {0, 0, 0, 0, 0, 0, 0, 0, -1};
  uint32_t carry = 0;
  // blkstat loads first: they are independent of the tile rounds
  uint32_t s5 = 0, s6 = 0, s7 = 0;
  for (int b0 = 0; b0 < nblk; b0 += 4 * kBig) {
    uint32_t a[4], z[4], y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int b = b0 + k * kBig + tid;
      a[k] = b < nblk ? blkstat[kBlkStats * b] : 0u;
      z[k] = b < nblk ? blkstat[kBlkStats * b + 1] : 0u;
      y[k] = b < nblk ? blkstat[kBlkStats * b + 2] : 0u;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      s5 += a[k];
      s6 += z[k];
      s7 += y[k];
    }
  }
  acc[5] = s5;
  acc[6] = s6;
  acc[7] = s7;
  for (int r0 = 0; r0 < T; r0 += kRound) {
    uint32_t v[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int p = tid + kBig * k, t = r0 + p;
      v[k] = t < T ? tot[t] : 0u;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int p = tid + kBig * k;
      stage[(p / kPer) * (kPer + 1) + p % kPer] = v[k];
    }
    __syncthreads();
    uint32_t w[kPer], run = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t c = stage[tid * (kPer + 1) + i];
      w[i] = c;
      run += c;
      acc[0] = acc[0] > (int64_t)c ? acc[0] : (int64_t)c;
      acc[1] += c > (uint32_t)kBlock;
      acc[2] += c > (uint32_t)kBlock ? c - kBlock : 0;
      acc[3] += c > (uint32_t)kMaxTileEntries;
      acc[4] += c > (uint32_t)kMaxTileEntries ? c - kMaxTileEntries : 0;
    }
    uint32_t round_total;
    uint32_t pos = carry + block_excl_scan<kBig>(run, &round_total);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      stage[tid * (kPer + 1) + i] = pos;
      if (w[i] > 0) {  // its last chunk: min(ceil(count / 512), 8) chunks of 512
        const int64_t last = (int64_t)pos + (int64_t)kBlock * (((w[i] < (uint32_t)kMaxTileEntries ? w[i]
                                                                 : (uint32_t)kMaxTileEntries) - 1) / kBlock);
        acc[8] = acc[8] > last ? acc[8] : last;
      }
      pos += w[i];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int p = tid + kBig * k, t = r0 + p;
      if (t < T) ranges[t] = (int32_t)stage[(p / kPer) * (kPer + 1) + p % kPer];
    }
    carry += round_total;
    __syncthreads();  // the stage is rewritten by the next round
  }
  // reduce the 9 accumulators over the block (0 and 8: maxima)
  const int lane = tid & 63, wid = tid >> 6;
#pragma unroll
  for (int k = 0; k < 9; ++k) {
    int64_t x = acc[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const int64_t y = __shfl_xor(x, o, 64);
      x = (k == 0 || k == 8) ? (x > y ? x : y) : x + y;
    }
    if (lane == 0) red[k][wid] = x;
  }
  __syncthreads();
  if (tid == 0) {
    int64_t r[9] = {0, 0, 0, 0, 0, 0, 0, 0, -1};
    for (int w = 0; w < kBig / 64; ++w)
      for (int k = 0; k < 9; ++k)
        r[k] = (k == 0 || k == 8) ? (r[k] > red[k][w] ? r[k] : red[k][w]) : r[k] + red[k][w];
    const int64_t m = carry;
    // the reference counts the valid slots of negative-depth Gaussians too (tile -1)
    const int64_t n_int = m + r[7];
    ranges[T] = (int32_t)m;
    for (int k = 0; k < GS_NUM_STATS; ++k) stats[k] = 0;
    stats[GS_STAT_N_INTERACTIONS] = (int32_t)n_int;
    stats[GS_STAT_TILE_ENTRIES] = (int32_t)m;
    stats[GS_STAT_MAX_PER_TILE] = (int32_t)r[0];
    stats[GS_STAT_OVERFLOW_TILES] = (int32_t)r[1];
    stats[GS_STAT_OVERFLOW_INTERACTIONS] = (int32_t)r[2];
    stats[GS_STAT_TRUNCATED_TILES] = (int32_t)r[3];
    stats[GS_STAT_TRUNCATED_INTERACTIONS] = (int32_t)r[4];
    stats[GS_STAT_RADIUS_CAP_VIOLATIONS] = (int32_t)r[5];
    stats[GS_STAT_NEGATIVE_DEPTH] = (int32_t)r[6];
    stats[GS_STAT_CAPACITY_EXCEEDED] = m > cap ? 1 : 0;
    // the reference's arrays hold max(256 n, 512) slots with 256 per negative-depth
    // Gaussian in front of the entries: a chunk starting past L - 512 there is clamped
    const int64_t L = 256 * n_gauss > kBlock ? 256 * n_gauss : kBlock;
    const bool clamped = r[8] >= 0 && 256 * r[6] + r[8] > L - kBlock;
    stats[GS_STAT_WINDOW_CLAMPED] = clamped ? 1 : 0;
    stats[GS_STAT_ENTRIES_DEFERRED] = deferred && defer_entries(T, m, cap, clamped) ? 1 : 0;
    // renderer.py:81: float32(n_interactions) / num_tiles
    stats[GS_STAT_MEAN_PER_TILE] = (int32_t)float_to_bits((float)(int32_t)n_int / (float)T);
  }
}

// 4b. Chunk offsets per tile (lane), in two levels so that a superblock with
// thousands of chunks (a dense cluster) is spread over many waves: the counting sweep
// adds each chunk's counts into its segment's totals (segments of kSeg chunks); one
// block per superblock turns its segments' totals into exclusive prefixes (in place)
// and writes the tile totals; the write sweep adds the counts of the chunk's earlier
// chunks in its segment.
// One block per superblock over its segments: 16 waves split them into contiguous
// runs, sum, scan the 16 run sums, then write the prefixes.
__global__ __launch_bounds__(kBig) void chunk_scan_kernel(const uint32_t* __restrict__ seg_base, int64_t gmax,
                                                          int SX, int TX, int TY, uint32_t* __restrict__ seg_sum,
                                                          uint32_t* __restrict__ tot) {
  constexpr int NW = kBig / 64;
  __shared__ uint32_t part[NW][64];
  const int sb = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint32_t g0 = seg_base[sb];
  const uint32_t g1 = (int64_t)seg_base[sb + 1] < gmax ? seg_base[sb + 1] : (uint32_t)gmax;
  const uint32_t per = g1 > g0 ? (g1 - g0 + NW - 1) / NW : 0u;
  const uint32_t a = g0 + wid * per < g1 ? g0 + wid * per : g1;
  const uint32_t b = a + per < g1 ? a + per : g1;
  uint32_t sum = 0;
#pragma unroll 8
  for (uint32_t g = a; g < b; ++g) sum += seg_sum[(int64_t)g * 64 + lane];
  part[wid][lane] = sum;
  __syncthreads();
  if (wid == 0) {
    uint32_t run = 0;
    for (int w = 0; w < NW; ++w) {
      const uint32_t v = part[w][lane];
      part[w][lane] = run;
      run += v;
    }
    const int t = tile_of(sb % SX, sb / SX, lane, TX, TY);
    if (t >= 0) tot[t] = run;
  }
  __syncthreads();
  uint32_t run = part[wid][lane];
  for (uint32_t g = a; g < b; ++g) {
    const uint32_t v = seg_sum[(int64_t)g * 64 + lane];
    seg_sum[(int64_t)g * 64 + lane] = run;
    run += v;
  }
}

// The window of gs_bin's compact list (gs_window_t): slots L-512..L-1 of the reference's
// L = max(256 n, 512)-slot arrays, laid out as gs_bin_reference writes them (negative-depth
// Gaussians' runs, the entries, the other Gaussians' empty slots in (dq, id) order,
// padding).  A chunk of the default path reads them only when the binning's stats set
// GS_STAT_WINDOW_CLAMPED, which needs fewer than 511 empty slots in all: then at most 510
// Gaussians have any, and the window's negative-depth runs are those of the last two
// negative-depth Gaussians in (dq, id) order.  One workgroup rebuilds them from the inputs.

// the larger two of (a0 >= a1) and (b0 >= b1), keys offset by one (0: none)
__device__ inline void top2_merge(uint64_t& a0, uint64_t& a1, uint64_t b0, uint64_t b1) {
  const uint64_t hi = a0 > b0 ? a0 : b0, lo = a0 > b0 ? b0 : a0;
  const uint64_t r1 = a1 > b1 ? a1 : b1;
  a0 = hi;
  a1 = lo > r1 ? lo : r1;
}

// The window, with the NT threads of one workgroup (every thread calls it): thr always, the
// ids when the stats say a chunk is clamped.
template <int NT>
__device__ void window_build(int64_t n, const float* __restrict__ means2d, const float* __restrict__ radii,
                             const uint8_t* __restrict__ valid, const float* __restrict__ depths, int W, int H,
                             const int32_t* __restrict__ gids, int64_t capacity, const int32_t* __restrict__ stats,
                             gs_window_t* __restrict__ win) {
  __shared__ uint64_t key[kBlock];
  __shared__ uint32_t cnt[kBlock], pre[kBlock];
  __shared__ uint64_t top_s[2 * (NT / 64)];
  __shared__ int n_tail;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t L = 256 * n > kBlock ? 256 * n : kBlock, lo = L - kBlock;
  const int64_t n_neg = stats[GS_STAT_NEGATIVE_DEPTH], m = stats[GS_STAT_TILE_ENTRIES];
  if (tid == 0) win->thr = lo - 256 * n_neg;
  if (tid < 2) win->reserved[tid] = 0;
  if (stats[GS_STAT_WINDOW_CLAMPED] == 0) return;  // no chunk reads the ids
  if (tid == 0) n_tail = 0;
  __syncthreads();
  // Gaussians with empty slots (non-negative depth), and the top two negative-depth ones
  uint64_t t0 = 0, t1 = 0;
  for (int64_t i = tid; i < n; i += NT) {
    const uint32_t zb = float_to_bits(depths[i]);
    const uint64_t k = ((uint64_t)depth_key(zb) << 32) | (uint64_t)i;
    if (zb >> 31) {
      top2_merge(t0, t1, k + 1, 0);
    } else {
      const TileRect t = tile_rect(means2d[2 * i], means2d[2 * i + 1], radii[i], valid[i] != 0, W, H);
      const uint32_t e = 256u - (uint32_t)t.count();
      if (e > 0) {
        const int at = atomicAdd(&n_tail, 1);
        if (at < kBlock) {
          key[at] = k;
          cnt[at] = e;
        }
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t b0 = __shfl_xor(t0, o, 64), b1 = __shfl_xor(t1, o, 64);
    top2_merge(t0, t1, b0, b1);
  }
  if (lane == 0) {
    top_s[2 * wid] = t0;
    top_s[2 * wid + 1] = t1;
  }
  __syncthreads();
  const int nt = n_tail < kBlock ? n_tail : kBlock;
  for (int i = tid; i < kBlock; i += NT)
    if (i >= nt) {
      key[i] = ~0ull;
      cnt[i] = 0;
    }
  __syncthreads();
  // bitonic sort of the (dq, id) keys, ascending
  for (int k = 2; k <= kBlock; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < kBlock; i += NT) {  // pairs (i, i ^ j) are disjoint within a step
        const int x = i ^ j;
        if (x > i) {
          const bool up = (i & k) == 0;
          if ((key[i] > key[x]) == up) {
            const uint64_t tk = key[i];
            key[i] = key[x];
            key[x] = tk;
            const uint32_t tc = cnt[i];
            cnt[i] = cnt[x];
            cnt[x] = tc;
          }
        }
      }
      __syncthreads();
    }
  if (tid == 0) {
    uint32_t acc = 0;
    for (int i = 0; i < kBlock; ++i) {
      pre[i] = acc;
      acc += cnt[i];
    }
    t0 = 0;
    t1 = 0;
    for (int w = 0; w < NT / 64; ++w) top2_merge(t0, t1, top_s[2 * w], top_s[2 * w + 1]);
    top_s[0] = t0;
    top_s[1] = t1;
  }
  __syncthreads();
  for (int i = tid; i < kBlock; i += NT) {
    const int64_t q = lo + i;
    int32_t id = 0;
    if (q < 256 * n_neg) {
      // rank q / 256 of the n_neg runs; the last two are top_s[1], top_s[0]
      const int64_t d = n_neg - 1 - q / 256;
      const uint64_t k = d == 0 ? top_s[0] : (d == 1 ? top_s[1] : 0);
      id = k ? (int32_t)(uint32_t)(k - 1) : 0;
    } else if (q < 256 * n_neg + m) {
      const int64_t e = q - 256 * n_neg;
      id = e < capacity ? gids[e] : 0;
    } else if (q < 256 * n) {
      const uint32_t u = (uint32_t)(q - 256 * n_neg - m);
      int a = 0, b = nt - 1;  // last sorted Gaussian whose run starts at or before u
      while (a < b) {
        const int c = (a + b + 1) >> 1;
        if (pre[c] <= u) a = c; else b = c - 1;
      }
      id = nt > 0 ? (int32_t)(uint32_t)key[a] : 0;
    }
    win->ids[i] = id;
  }
}


// gs_window_from_bins: the window on its own (one workgroup).
constexpr int kWinThreads = 1024;
__global__ __launch_bounds__(kWinThreads) void window_bins_kernel(
    int64_t n, const float* __restrict__ means2d, const float* __restrict__ radii, const uint8_t* __restrict__ valid,
    const float* __restrict__ depths, int W, int H, const int32_t* __restrict__ gids, int64_t capacity,
    const int32_t* __restrict__ stats, gs_window_t* __restrict__ win) {
  window_build<kWinThreads>(n, means2d, radii, valid, depths, W, H, gids, capacity, stats, win);
}

// 4d. write every entry: tile t's entries from chunk c start at ranges[t] plus the
// counts of the superblock's earlier chunks; within a step the 64 tiles are visited
// in an unrolled loop with wave-uniform masks (column & row ballots), and the lanes
// of a tile's mask store their ids at base + popcount(mask & lanes-below): one
// contiguous run per store.  Lane u holds tile u's next slot (read with v_readlane,
// advanced once per step).  A chunk costs two memory round trips: its descriptor
// (with its counts), then its 256 words and the tiles' range starts together.
// CHECK: some entries fall beyond the capacity and are dropped.
template <bool WITH_TILES, bool CHECK>
__device__ inline void write_step(uint64_t word, bool act, int sx, int sy, int lane, uint32_t n_gauss, int TX,
                                  uint32_t cap32, uint32_t& base, int32_t* __restrict__ out_gid,
                                  int32_t* __restrict__ out_tile) {
  const Packed g = unpack(act ? word : 0ull);
  act = act && g.gid < n_gauss;  // ids are < n by construction
  // column and row masks are wave-uniform; tile (ux, uy)'s mask is their AND
  uint64_t cm[kSB], rm[kSB];
#pragma unroll
  for (int k = 0; k < kSB; ++k) {
    const int tx = sx * kSB + k, ty = sy * kSB + k;
    cm[k] = __ballot(act && g.x0 <= tx && tx < g.x0 + g.w);
    rm[k] = __ballot(act && g.y0 <= ty && ty < g.y0 + g.h);
  }
#pragma unroll
  for (int uy = 0; uy < kSB; ++uy) {
    if (rm[uy] == 0ull) continue;
#pragma unroll
    for (int ux = 0; ux < kSB; ++ux) {
      const uint64_t m = cm[ux] & rm[uy];
      if (m == 0ull) continue;
      const uint32_t b = __builtin_amdgcn_readlane(base, uy * kSB + ux);
      if (__builtin_amdgcn_inverse_ballot_w64(m)) {
        // lanes of m store their ids at b + (lanes of m below them): one run
        const uint32_t dst =
            b + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (!CHECK || dst < cap32) {
          out_gid[dst] = (int32_t)g.gid;
          if (WITH_TILES) out_tile[dst] = (sy * kSB + uy) * TX + sx * kSB + ux;
        }
      }
    }
  }
  // lane u advances tile u's slot by its count in this step
  uint64_t mine = 0;
  const int ux = lane & 7, uy = lane >> 3;
#pragma unroll
  for (int k = 0; k < kSB; ++k) mine = ux == k ? cm[k] : mine;
  uint64_t rmine = 0;
#pragma unroll
  for (int k = 0; k < kSB; ++k) rmine = uy == k ? rm[k] : rmine;
  base += (uint32_t)__popcll(mine & rmine);
}

template <bool WITH_TILES, bool CHECK>
__device__ inline void write_chunk(const uint4& d, const uint64_t* __restrict__ pval, uint32_t n_gauss, int TX, int TY,
                                   uint32_t cnt_c, const uint32_t* __restrict__ seg_pre,
                                   const int32_t* __restrict__ ranges, uint32_t cap32, int lane,
                                   int32_t* __restrict__ out_gid, int32_t* __restrict__ out_tile) {
  const int len = (int)(d.y & 0xFFFFu), sx = (int)(d.z & 0xFFFFu), sy = (int)(d.z >> 16);
  const int t = tile_of(sx, sy, lane, TX, TY);
  uint64_t wv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) wv[k] = 64 * k + lane < len ? pval[d.x + 64 * k + lane] : 0ull;
  // lane u: next slot of tile u (tiles outside the image never get entries): the
  // tile's range start + the superblock's earlier segments + earlier chunks of this one
  uint32_t base = (t >= 0 ? (uint32_t)ranges[t] : 0u) + seg_pre[(int64_t)d.w * 64 + lane] + cnt_c;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (64 * k < len)
      write_step<WITH_TILES, CHECK>(wv[k], 64 * k + lane < len, sx, sy, lane, n_gauss, TX, cap32, base, out_gid,
                                    out_tile);
}

// The default path's chunk window of the list being written (NULL win: none), with the
// binning's inputs its clamped form is rebuilt from.
struct WinArgs {
  gs_window_t* win;
  const float* means2d;
  const float* radii;
  const uint8_t* valid;
  const float* depths;
  int W, H;
  uint32_t* ticket;  // finished workgroups of the sweep (cleared by the tile scan)
};

// OFFSET: the entries go after the 256 slots of every negative-depth Gaussian (the
// reference's full arrays): the outputs start at 256 * stats[GS_STAT_NEGATIVE_DEPTH],
// which tile_scan_stats_kernel has written.
// DEFER (gs_bin_deferred): nothing is written when entries_deferred holds; the compositing
// forward then writes the entries it meets.
// The window (wa.win): its threshold from workgroup 0 at the start; when a chunk is clamped
// (never with a deferred list), its ids from the last workgroup to finish, once every entry
// is written (each workgroup's entries made visible device-wide before it counts itself
// finished), which saves the window its own launch.
template <bool WITH_TILES, bool OFFSET, bool DEFER>
__global__ __launch_bounds__(256) void tile_write_kernel(const uint32_t* __restrict__ n_chunks, int64_t cmax,
                                                         const uint4* __restrict__ desc,
                                                         const uint64_t* __restrict__ pval, uint32_t n_gauss, int TX,
                                                         int TY, const uint32_t* __restrict__ cnt,
                                                         const uint32_t* __restrict__ seg_pre,
                                                         const int32_t* __restrict__ ranges, int T, int64_t cap,
                                                         int32_t* __restrict__ out_gid,
                                                         int32_t* __restrict__ out_tile,
                                                         const int32_t* __restrict__ stats, const WinArgs wa) {
  const int32_t* const gids_in = out_gid;  // the list as the window reads it (no offset)
  const int64_t cap_in = cap;
  bool clamped = false;
  if constexpr (!OFFSET) {
    clamped = wa.win != nullptr && stats[GS_STAT_WINDOW_CLAMPED] != 0;
    if (wa.win != nullptr && !clamped && blockIdx.x == 0)  // the threshold only (no chunk reads ids)
      window_build<256>(n_gauss, wa.means2d, wa.radii, wa.valid, wa.depths, wa.W, wa.H, gids_in, cap_in, stats,
                        wa.win);
  }
  if (DEFER && entries_deferred(stats)) return;
  const int lane = threadIdx.x & 63;
  const uint32_t nwaves = gridDim.x * (blockDim.x / 64);
  const uint32_t C = (uint32_t)min<int64_t>((int64_t)*n_chunks, cmax);
  if (OFFSET) {
    const int64_t off = 256 * (int64_t)stats[GS_STAT_NEGATIVE_DEPTH];
    out_gid += off;
    if (WITH_TILES) out_tile += off;
    cap -= off;  // >= the entry count: every Gaussian's entries fit in its 256 slots
  }
  const uint32_t cap32 = (uint32_t)cap;  // gs_bin checks cap < 2^31
  // every entry fits (the usual case): no per-store capacity test
  const bool fits = ranges[T] >= 0 && (int64_t)ranges[T] <= cap;
  for (uint32_t c = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); c < C; c += nwaves) {
    const uint4 d = desc[c];
    // counts of the chunk's earlier chunks in its segment (p of them), loaded together
    const uint32_t p = d.y >> 16;
    uint32_t cnt_c = 0;
#pragma unroll
    for (int k = 1; k < kSeg; ++k) cnt_c += (uint32_t)k <= p ? cnt[(int64_t)(c - k) * 64 + lane] : 0u;
    if (fits)
      write_chunk<WITH_TILES, false>(d, pval, n_gauss, TX, TY, cnt_c, seg_pre, ranges, cap32, lane, out_gid, out_tile);
    else
      write_chunk<WITH_TILES, true>(d, pval, n_gauss, TX, TY, cnt_c, seg_pre, ranges, cap32, lane, out_gid, out_tile);
  }
  if constexpr (!OFFSET) {
    if (clamped) {  // (uniform: every workgroup takes this branch or none)
      __shared__ int last;
      __threadfence();  // this thread's entries, visible device-wide
      __syncthreads();
      if (threadIdx.x == 0) last = atomicAdd(wa.ticket, 1u) == gridDim.x - 1;
      __syncthreads();
      if (last) {
        __threadfence();  // and every other workgroup's, seen here
        window_build<256>(n_gauss, wa.means2d, wa.radii, wa.valid, wa.depths, wa.W, wa.H, gids_in, cap_in, stats,
                          wa.win);
      }
    }
  }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------------
struct BinPlan {
  int64_t n, cap, pcap, cmax, gmax;
  int T, TX, TY, SX, SY, S;
  int G_d;        // depth-sort workgroups (= bin_prep blocks)
  int G_q;        // workgroups of the first superblock pass
  int G_p;        // workgroups of the second pair pass
  int sb_passes;  // 1 when S <= 256, else 2
  size_t o_dkey, o_word, o_ka, o_wa, o_kb, o_wb, o_table, o_dtot, o_scal, o_pk0, o_pv0, o_pk1, o_pv1, o_sbr,
      o_cbase, o_csb, o_cnt, o_desc, o_tot, o_blk, o_gbase, o_gsum, o_masks, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// deferred: room for the count sweep's tile masks (gs_bin_deferred)
BinPlan make_plan(int64_t n, int width, int height, int64_t capacity, bool deferred = false) {
  BinPlan P;
  P.n = n;
  P.cap = capacity > 0 ? capacity : 256 * (n > 2 ? n : 2);
  P.TX = (width + kTile - 1) / kTile;
  P.TY = (height + kTile - 1) / kTile;
  P.T = P.TX * P.TY;
  P.SX = (P.TX + kSB - 1) / kSB;
  P.SY = (P.TY + kSB - 1) / kSB;
  P.S = P.SX * P.SY;
  P.sb_passes = P.S <= (1 << kPairRB) ? 1 : 2;
  const int64_t nn = std::max<int64_t>(n, 1);
  P.pcap = (int64_t)kSBSpan * kSBSpan * nn;
  P.cmax = (P.pcap + kChunk - 1) / kChunk + P.S;
  P.gmax = (P.cmax + kSeg - 1) / kSeg + P.S;
  P.G_d = (int)((nn + kSpan - 1) / kSpan);
  P.G_q = (int)((nn + kPairSpan - 1) / kPairSpan);
  P.G_p = (int)std::min<int64_t>(8192, std::max<int64_t>(1, (2 * nn + 1023) / 1024));
  const int64_t tbl = (int64_t)(1 << kPairRB) * std::max(P.G_q, P.G_p);
  const bool two = P.sb_passes == 2;
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
  P.o_table = take((size_t)tbl * 4);
  P.o_dtot = take((1 << kPairRB) * 4);
  P.o_scal = take(256);  // device scalars: [0] pairs, [1] chunks
  P.o_pk0 = take(two ? (size_t)P.pcap * 4 : 0);
  P.o_pv0 = take((size_t)P.pcap * 8);
  P.o_pk1 = take(two ? (size_t)P.pcap * 4 : 0);
  P.o_pv1 = take(two ? (size_t)P.pcap * 8 : 0);
  P.o_sbr = take(((size_t)P.S + 1) * 4);
  P.o_cbase = take(((size_t)P.S + 1) * 4);
  P.o_csb = take((size_t)P.cmax * 4);
  P.o_cnt = take((size_t)P.cmax * 64 * 4);
  P.o_desc = take((size_t)P.cmax * 16);
  P.o_tot = take((size_t)P.T * 4);
  P.o_blk = take((size_t)P.G_d * kBlkStats * 4);
  P.o_gbase = take(((size_t)P.S + 1) * 4);
  P.o_gsum = take((size_t)P.gmax * 64 * 4);
  P.o_masks = take(deferred ? (size_t)P.cmax * 64 * (kChunk / 64) * 8 : 0);  // [chunk][tile][step]
  P.total = o;
  return P;
}

// One stable radix pass: keys_in/vals_in -> keys_out/vals_out on digit `shift`.
// The upsweep is skipped when the table was already filled.
template <int RB>
int radix_pass(hipStream_t s, bool upsweep, const uint32_t* kin, const uint64_t* vin, uint32_t* kout, uint64_t* vout,
               const uint32_t* n_dev, int64_t n_static, int64_t cap, int shift, int G, int fixed_chunk,
               uint32_t* table, uint32_t* dtot, bool drop_empty = false, uint32_t* n_kept = nullptr) {
  if (upsweep) {
    hipLaunchKernelGGL(radix_upsweep_kernel<RB>, dim3(G), dim3(64), 0, s, kin, n_dev, n_static, cap, shift, G,
                       fixed_chunk, table);
    GS_LAUNCH_CHECK("radix_upsweep_kernel");
  }
  hipLaunchKernelGGL(radix_spine_kernel, dim3(1 << RB), dim3(kScanBlock), 0, s, table, G, dtot);
  GS_LAUNCH_CHECK("radix_spine_kernel");
  hipLaunchKernelGGL(radix_downsweep_kernel<RB>, dim3(G), dim3(64), 0, s, kin, vin, n_dev, n_static, cap, shift, G,
                     fixed_chunk, table, dtot, kout, vout, drop_empty, n_kept);
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

extern "C" size_t gs_bin_deferred_workspace_size(int64_t n, int width, int height, int64_t capacity) {
  if (n < 0 || width <= 0 || height <= 0) return 0;
  return make_plan(n, width, height, capacity, true).total;
}

namespace gs {
namespace {
int bin_run(void* stream, int64_t n, const float* means2d, const float* radii, const uint8_t* valid,
            const float* depths, int width, int height, int64_t capacity, void* workspace, size_t workspace_bytes,
            int32_t* sorted_gids, int32_t* sorted_tiles, int32_t* ranges, int32_t* stats, bool ref_offset,
            bool deferred = false, gs_window_t* window = nullptr) {
  GS_REQUIRE(n >= 0 && n <= ((int64_t)1 << 26), "gs_bin: n must be in [0, 2^26] (got %lld)", (long long)n);
  GS_REQUIRE(width > 0 && height > 0 && width <= 4096 * kTile && height <= 4096 * kTile,
             "gs_bin: bad image size %dx%d (each side at most 65536)", width, height);
  const BinPlan P = make_plan(n, width, height, capacity, deferred);
  GS_REQUIRE(P.cap < ((int64_t)1 << 31), "gs_bin: capacity %lld too large", (long long)P.cap);
  GS_REQUIRE(P.S <= (1 << (2 * kPairRB)), "gs_bin: %d tiles exceed the supported 65536 superblocks of 8x8 tiles",
             P.T);
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
  uint4* desc = (uint4*)(ws + P.o_desc);
  uint32_t* tot = (uint32_t*)(ws + P.o_tot);
  uint32_t* blk = (uint32_t*)(ws + P.o_blk);
  uint32_t* gbase = (uint32_t*)(ws + P.o_gbase);
  uint32_t* gsum = (uint32_t*)(ws + P.o_gsum);
  uint64_t* masks = deferred ? (uint64_t*)(ws + P.o_masks) : nullptr;
  uint32_t* n_pairs = scal + 0;
  uint32_t* n_chunks = scal + 1;
  uint32_t* n_segs = scal + 2;
  uint32_t* n_has = scal + 3;  // Gaussians that meet at least one tile
  uint32_t* ticket = scal + 4;  // workgroups of the write sweep done (the window's last one builds it)

  if (n == 0) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, s, stats, (int64_t)GS_NUM_STATS, 0);
    GS_LAUNCH_CHECK("fill_i32_kernel");
    hipLaunchKernelGGL(fill_i32_kernel, dim3(div_up(P.T + 1, 256)), dim3(256), 0, s, ranges, (int64_t)P.T + 1, 0);
    GS_LAUNCH_CHECK("fill_i32_kernel");
    if (window != nullptr) {
      hipLaunchKernelGGL(window_bins_kernel, dim3(1), dim3(kWinThreads), 0, s, n, means2d, radii, valid, depths,
                         width, height, sorted_gids, P.cap, stats, window);
      GS_LAUNCH_CHECK("window_bins_kernel");
    }
    return GS_OK;
  }
  // 1. prep (+ histogram of the first depth digit)
  hipLaunchKernelGGL(bin_prep_kernel, dim3(P.G_d), dim3(kPrepBlock), 0, s, n, means2d, radii, valid, depths,
                     width, height, P.G_d, dkey, word, table, blk, (uint4*)gsum, P.gmax * 64 / 4);
  GS_LAUNCH_CHECK("bin_prep_kernel");
  // 2. stable depth sort of the packed words (13-bit bucket: 7 + 6 bits)
  // (the first pass drops Gaussians that meet no tile; the later passes see n_has)
  int rc = radix_pass<kDepthRB>(s, false, dkey, word, kb, wb, nullptr, n, n, 0, P.G_d, kSpan, table, dtot, true,
                                n_has);
  if (rc != GS_OK) return rc;
  rc = radix_pass<kDepthRB>(s, true, kb, wb, ka, wa, n_has, n, n, kDepthRB, P.G_d, kSpan, table, dtot);
  if (rc != GS_OK) return rc;
  const uint64_t* sorted_word = wa;
  // 3. superblock pairs generated from the depth order, sorted by superblock
  hipLaunchKernelGGL(pair_upsweep_kernel, dim3(div_up(P.G_q, 8) * 8), dim3(256), 0, s, sorted_word, n, n_has, P.SX,
                     P.G_q, table);
  GS_LAUNCH_CHECK("pair_upsweep_kernel");
  hipLaunchKernelGGL(radix_spine_kernel, dim3(1 << kPairRB), dim3(kScanBlock), 0, s, table, P.G_q, dtot);
  GS_LAUNCH_CHECK("radix_spine_kernel");
  const uint64_t* sbval = pv0;
  ChunkMapArgs maps{0, P.cmax, P.gmax, sbr, cbase, csb, n_chunks, gbase, n_segs};
  if (P.sb_passes == 1) {
    maps.S = P.S;  // one superblock pass: the pass also builds the chunk maps
    hipLaunchKernelGGL(pair_downsweep_kernel<false>, dim3(P.G_q), dim3(64), 0, s, sorted_word, n, n_has, P.SX, P.G_q,
                       table,
                       dtot, nullptr, pv0, n_pairs, maps);
    GS_LAUNCH_CHECK("pair_downsweep_kernel");
  } else {
    hipLaunchKernelGGL(pair_downsweep_kernel<true>, dim3(P.G_q), dim3(64), 0, s, sorted_word, n, n_has, P.SX, P.G_q,
                       table,
                       dtot, pk0, pv0, n_pairs, maps);
    GS_LAUNCH_CHECK("pair_downsweep_kernel");
    rc = radix_pass<kPairRB>(s, true, pk0, pv0, pk1, pv1, n_pairs, 0, P.pcap, kPairRB, P.G_p, 0, table, dtot);
    if (rc != GS_OK) return rc;
    sbval = pv1;
    hipLaunchKernelGGL(ranges_kernel, dim3(std::min(2048, div_up(P.pcap + 1, 256))), dim3(256), 0, s, pk1, n_pairs,
                       P.pcap, P.S, sbr);
    GS_LAUNCH_CHECK("ranges_kernel");
  }
  // 4. tile pass
  if (P.sb_passes != 1) {  // (one pass: built by the superblock pass)
    hipLaunchKernelGGL(chunks_kernel, dim3(1), dim3(kBig), 0, s, P.S, sbr, P.cmax, cbase, csb, n_chunks, P.gmax,
                       gbase, n_segs);
    GS_LAUNCH_CHECK("chunks_kernel");
  }
  // one chunk per wave: the chunk count is known on the device only, so the grid covers
  // the bound and surplus waves exit at once; waves start as others finish
  const int pass_blocks = (int)std::min<int64_t>(div_up(P.cmax, 4), (int64_t)1 << 20);
  hipLaunchKernelGGL(tile_count_kernel, dim3(pass_blocks), dim3(256), 0, s, n_chunks, P.cmax, csb, cbase, sbr, P.S,
                     sbval, P.SX, gbase, cnt, desc, gsum, masks);
  GS_LAUNCH_CHECK("tile_count_kernel");
  hipLaunchKernelGGL(chunk_scan_kernel, dim3(P.S), dim3(kBig), 0, s, gbase, P.gmax, P.SX, P.TX, P.TY, gsum, tot);
  GS_LAUNCH_CHECK("chunk_scan_kernel");
  hipLaunchKernelGGL(tile_scan_stats_kernel, dim3(1), dim3(kBig), 0, s, tot, P.T, blk, P.G_d, P.cap, n, ranges,
                     stats, deferred, ticket);
  GS_LAUNCH_CHECK("tile_scan_stats_kernel");
  // the deferred sweep usually exits at once: a smaller grid (its loop covers every chunk)
  const int write_blocks = deferred ? std::min(pass_blocks, 1024) : pass_blocks;
  const WinArgs winargs{ref_offset ? nullptr : window, means2d, radii, valid, depths, width, height, ticket};
#define GS_WRITE_LAUNCH(TILES, OFF, DEFER)                                                                      \
  hipLaunchKernelGGL((tile_write_kernel<TILES, OFF, DEFER>), dim3(write_blocks), dim3(256), 0, s, n_chunks, P.cmax, \
                     desc, sbval, (uint32_t)n, P.TX, P.TY, cnt, gsum, ranges, P.T, P.cap, sorted_gids, sorted_tiles, \
                     stats, winargs)
  if (ref_offset)
    GS_WRITE_LAUNCH(true, true, false);
  else if (sorted_tiles != nullptr)
    GS_WRITE_LAUNCH(true, false, false);
  else if (deferred)
    GS_WRITE_LAUNCH(false, false, true);
  else
    GS_WRITE_LAUNCH(false, false, false);
#undef GS_WRITE_LAUNCH
  GS_LAUNCH_CHECK("tile_write_kernel");
  return GS_OK;
}
}  // namespace
}  // namespace gs

extern "C" int gs_bin(void* stream, int64_t n, const float* means2d, const float* radii, const uint8_t* valid,
                      const float* depths, int width, int height, int64_t capacity, void* workspace,
                      size_t workspace_bytes, int32_t* sorted_gids, int32_t* sorted_tiles, int32_t* ranges,
                      int32_t* stats, gs_window_t* window) {
  return bin_run(stream, n, means2d, radii, valid, depths, width, height, capacity, workspace, workspace_bytes,
                 sorted_gids, sorted_tiles, ranges, stats, false, false, window);
}

extern "C" int gs_bin_deferred(void* stream, int64_t n, const float* means2d, const float* radii,
                               const uint8_t* valid, const float* depths, int width, int height, int64_t capacity,
                               void* workspace, size_t workspace_bytes, int32_t* sorted_gids, int32_t* ranges,
                               int32_t* stats, gs_window_t* window) {
  return bin_run(stream, n, means2d, radii, valid, depths, width, height, capacity, workspace, workspace_bytes,
                 sorted_gids, nullptr, ranges, stats, false, true, window);
}

namespace gs {
int superblock_lists(int64_t n, int width, int height, int64_t capacity, const void* workspace,
                     size_t workspace_bytes, const int32_t* stats, SBLists* out) {
  GS_REQUIRE(n >= 0 && n <= ((int64_t)1 << 26) && width > 0 && height > 0 && width <= 4096 * kTile &&
                 height <= 4096 * kTile,
             "superblock lists: bad sizes (n %lld, %dx%d)", (long long)n, width, height);
  const BinPlan P = make_plan(n, width, height, capacity, true);
  GS_REQUIRE(workspace != nullptr && workspace_bytes >= P.total,
             "superblock lists: a workspace of %zu bytes is smaller than the binning's %zu", workspace_bytes,
             P.total);
  const char* ws = (const char*)workspace;
  out->words = (const uint64_t*)(ws + (P.sb_passes == 1 ? P.o_pv0 : P.o_pv1));
  out->ranges = (const int32_t*)(ws + P.o_sbr);
  out->chunk_base = (const uint32_t*)(ws + P.o_cbase);
  out->masks = (const uint64_t*)(ws + P.o_masks);
  out->n_chunks = P.cmax;
  out->n_words = P.pcap;
  out->SX = P.SX;
  out->stats = stats;
  return GS_OK;
}
}  // namespace gs

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

// ---------------------------------------------------------------------------------
// gs_bin_static: gs_bin with its workspace in a library-owned device array, for callers
// that cannot allocate.  Every GPU the library runs on holds its own copy of `scratch`
// (GS_BIN_STATIC_SCRATCH_BYTES) until the process ends.  Host code never passes the
// array's name to a kernel: its device address, per device, comes from
// hipGetSymbolAddress on the entry point's first call with that device current.
// gs_bin's kernels need no cleared workspace (whatever must start at zero is cleared
// by its first launch), so a call may follow any other on the same array; calls that
// overlap on one GPU (other streams or threads) share it and race.
static __device__ __align__(256) unsigned char scratch[GS_BIN_STATIC_SCRATCH_BYTES];

namespace gs {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(void** out) {
  int dev = -1;
  int rc = hip_check(hipGetDevice(&dev), "gs_bin_static: hipGetDevice");
  if (rc != GS_OK) return rc;
  GS_REQUIRE(dev >= 0 && dev < kMaxDevices, "gs_bin_static: device %d out of the supported range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    rc = hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "gs_bin_static: hipGetSymbolAddress");
    if (rc != GS_OK) return rc;
    GS_REQUIRE(ptr != nullptr, "gs_bin_static: no device address for the scratch array");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GS_OK;
}
}  // namespace
}  // namespace gs

extern "C" int gs_bin_static(void* stream, int64_t n, const float* means2d, const float* radii, const uint8_t* valid,
                             const float* depths, int width, int height, int64_t capacity, int32_t* sorted_gids,
                             int32_t* sorted_tiles, int32_t* ranges, int32_t* stats) {
  GS_REQUIRE(n >= 0 && width > 0 && height > 0, "gs_bin_static: bad sizes (n %lld, image %dx%d)", (long long)n,
             width, height);
  const size_t need = gs_bin_workspace_size(n, width, height, capacity);
  GS_REQUIRE(need <= (size_t)GS_BIN_STATIC_SCRATCH_BYTES,
             "gs_bin_static: %lld Gaussians on a %dx%d image need %zu bytes of workspace, more than the %zu of "
             "the static scratch array (use gs_bin with a caller workspace)",
             (long long)n, width, height, need, (size_t)GS_BIN_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_on_current_device(&ws);
  if (rc != GS_OK) return rc;
  return gs_bin(stream, n, means2d, radii, valid, depths, width, height, capacity, ws,
                (size_t)GS_BIN_STATIC_SCRATCH_BYTES, sorted_gids, sorted_tiles, ranges, stats, nullptr);
}

// ---------------------------------------------------------------------------------
// The reference's full arrays (rasterizer.py:84-114): all 256 n slots in the order of the
// stable sort of their keys (tile << 13) | dq, with dq the Gaussian's signed depth
// quantum and tile = T for a slot that holds no entry; a negative dq makes every key of
// its Gaussian negative (tile -1).  In order:
//   * the 256 slots of every negative-depth Gaussian, tile -1, Gaussians in (dq, id) order;
//   * the entries, tiles 0..T-1 (gs_bin's list, written there by the offset write sweep);
//   * the 256 - count empty slots of every other Gaussian, tile T, in (dq, id) order;
//   * when 256 n < 512, padding up to 512 with tile T and id 0 (rasterizer.py:107-114).
// The two runs of slots come from one stable sort of all Gaussians by dq (two 7-bit
// radix passes: negative quanta sort first) and a scan of their slot counts.
namespace gs {
namespace {

// per Gaussian: sort key dq + 8192 and value id | (slots << 32), slots = 256 for a
// negative depth, else 256 - (its entries)
__global__ __launch_bounds__(kPrepBlock) void ref_prep_kernel(int64_t n, const float* __restrict__ means2d,
                                                              const float* __restrict__ radii,
                                                              const uint8_t* __restrict__ valid,
                                                              const float* __restrict__ depths, int W, int H,
                                                              uint32_t* __restrict__ keys,
                                                              uint64_t* __restrict__ vals) {
  for (int r = 0; r < kPrepPer; ++r) {
    const int64_t i = (int64_t)blockIdx.x * kSpan + r * kPrepBlock + threadIdx.x;
    if (i >= n) continue;
    const TileRect t = tile_rect(means2d[2 * i], means2d[2 * i + 1], radii[i], valid[i] != 0, W, H);
    const uint32_t zb = float_to_bits(depths[i]);
    const uint32_t slots = (zb >> 31) ? 256u : 256u - (uint32_t)t.count();
    keys[i] = depth_key(zb);
    vals[i] = (uint64_t)i | ((uint64_t)slots << 32);
  }
}

// slots of the kSpan sorted Gaussians of each workgroup
__global__ __launch_bounds__(kPrepBlock) void ref_sum_kernel(int64_t n, const uint64_t* __restrict__ vals,
                                                             uint32_t* __restrict__ gsum) {
  uint32_t s = 0;
  for (int r = 0; r < kPrepPer; ++r) {
    const int64_t i = (int64_t)blockIdx.x * kSpan + r * kPrepBlock + threadIdx.x;
    if (i < n) s += (uint32_t)(vals[i] >> 32);
  }
  uint32_t tot;
  block_excl_scan<kPrepBlock>(s, &tot);
  if (threadIdx.x == 0) gsum[blockIdx.x] = tot;
}

// one block: exclusive scan of the G workgroup sums in place
__global__ __launch_bounds__(kBig) void ref_scan_kernel(uint32_t* __restrict__ gsum, int G) {
  uint32_t carry = 0;
  for (int r0 = 0; r0 < G; r0 += kBig) {
    const int g = r0 + threadIdx.x;
    const uint32_t v = g < G ? gsum[g] : 0u;
    uint32_t tot;
    const uint32_t ex = block_excl_scan<kBig>(v, &tot);
    if (g < G) gsum[g] = carry + ex;
    carry += tot;
    __syncthreads();
  }
}

// Each workgroup places its kSpan sorted Gaussians' runs: the first slot of a Gaussian is
// its workgroup's base plus the slots before it in the workgroup; Gaussians after the
// n_neg negative-depth ones also skip the entries.  Each wave writes the runs of every
// fourth Gaussian (at most 256 slots each).  Workgroup 0 also writes the padding and
// moves the tile ranges past the tile -1 slots.
__global__ __launch_bounds__(kPrepBlock) void ref_fill_kernel(int64_t n, const uint64_t* __restrict__ vals,
                                                              const uint32_t* __restrict__ gsum,
                                                              const int32_t* __restrict__ stats, int T, int64_t L,
                                                              int32_t* __restrict__ out_tiles,
                                                              int32_t* __restrict__ out_gids,
                                                              int32_t* __restrict__ ranges) {
  __shared__ uint32_t pos_s[kSpan], gid_s[kSpan];
  __shared__ uint16_t cnt_s[kSpan];
  const int tid = threadIdx.x;
  const int64_t b0 = (int64_t)blockIdx.x * kSpan;
  const int64_t n_neg = stats[GS_STAT_NEGATIVE_DEPTH];
  const uint32_t n_ent = (uint32_t)stats[GS_STAT_TILE_ENTRIES];
  static_assert(kSpan == 4 * kPrepBlock, "four consecutive Gaussians per thread");
  uint32_t e[4], g[4], run = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t i = b0 + 4 * tid + k;
    const uint64_t v = i < n ? vals[i] : 0ull;
    e[k] = (uint32_t)(v >> 32);
    g[k] = (uint32_t)v;
    run += e[k];
  }
  uint32_t tot;
  uint32_t p = gsum[blockIdx.x] + block_excl_scan<kPrepBlock>(run, &tot);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t i = b0 + 4 * tid + k;
    pos_s[4 * tid + k] = p + (i >= n_neg ? n_ent : 0u);
    gid_s[4 * tid + k] = g[k];
    cnt_s[4 * tid + k] = (uint16_t)e[k];
    p += e[k];
  }
  __syncthreads();
  const int lane = tid & 63, w = tid >> 6;
  for (int j = w; j < kSpan; j += kPrepBlock / 64) {
    const int64_t i = b0 + j;
    if (i >= n) break;
    const uint32_t c = cnt_s[j], base = pos_s[j];
    const int32_t gid = (int32_t)gid_s[j], tile = i < n_neg ? -1 : T;
    for (uint32_t q = lane; q < c; q += 64) {
      if ((int64_t)base + q >= L) break;  // never, for stats consistent with the slot counts
      out_gids[base + q] = gid;
      out_tiles[base + q] = tile;
    }
  }
  if (blockIdx.x == 0) {
    for (int64_t q = 256 * n + tid; q < L; q += kPrepBlock) {
      out_tiles[q] = T;
      out_gids[q] = 0;
    }
    for (int t = tid; t <= T; t += kPrepBlock) ranges[t] += (int32_t)(256 * n_neg);
  }
}

struct RefPlan {
  BinPlan bin;
  int64_t L;
  int G;
  size_t o_keys, o_vals, o_keys2, o_vals2, o_table, o_dtot, o_gsum, total;
};

RefPlan make_ref_plan(int64_t n, int width, int height) {
  RefPlan R;
  R.L = std::max<int64_t>(256 * n, kBlock);
  R.bin = make_plan(n, width, height, R.L);
  const int64_t nn = std::max<int64_t>(n, 1);
  R.G = (int)((nn + kSpan - 1) / kSpan);
  size_t o = R.bin.total;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align256(o + bytes);
    return at;
  };
  R.o_keys = take(nn * 4);
  R.o_vals = take(nn * 8);
  R.o_keys2 = take(nn * 4);
  R.o_vals2 = take(nn * 8);
  R.o_table = take((size_t)(1 << kDepthRB) * R.G * 4);
  R.o_dtot = take((1 << kDepthRB) * 4);
  R.o_gsum = take((size_t)R.G * 4);
  R.total = o;
  return R;
}

}  // namespace
}  // namespace gs

extern "C" size_t gs_bin_reference_workspace_size(int64_t n, int width, int height) {
  if (n < 0 || width <= 0 || height <= 0) return 0;
  return make_ref_plan(n, width, height).total;
}

extern "C" int gs_bin_reference(void* stream, int64_t n, const float* means2d, const float* radii,
                                const uint8_t* valid, const float* depths, int width, int height, void* workspace,
                                size_t workspace_bytes, int32_t* sorted_tiles, int32_t* sorted_gids, int32_t* ranges,
                                int32_t* stats) {
  GS_REQUIRE(n >= 0 && n < ((int64_t)1 << 23), "gs_bin_reference: n must be in [0, 2^23) (got %lld): the %s",
             (long long)n, "256 n slots are indexed with int32");
  GS_REQUIRE(width > 0 && height > 0, "gs_bin_reference: bad image size %dx%d", width, height);
  const RefPlan R = make_ref_plan(n, width, height);
  GS_REQUIRE(workspace != nullptr && workspace_bytes >= R.total,
             "gs_bin_reference: workspace of %zu bytes is smaller than the %zu required", workspace_bytes, R.total);
  GS_REQUIRE(sorted_tiles && sorted_gids && ranges && stats, "gs_bin_reference: NULL output");
  hipStream_t s = (hipStream_t)stream;
  int rc = bin_run(stream, n, means2d, radii, valid, depths, width, height, R.L, workspace, R.bin.total, sorted_gids,
                   sorted_tiles, ranges, stats, true);
  if (rc != GS_OK) return rc;
  char* ws = (char*)workspace;
  uint32_t* keys = (uint32_t*)(ws + R.o_keys);
  uint64_t* vals = (uint64_t*)(ws + R.o_vals);
  uint32_t* keys2 = (uint32_t*)(ws + R.o_keys2);
  uint64_t* vals2 = (uint64_t*)(ws + R.o_vals2);
  uint32_t* table = (uint32_t*)(ws + R.o_table);
  uint32_t* dtot = (uint32_t*)(ws + R.o_dtot);
  uint32_t* gsum = (uint32_t*)(ws + R.o_gsum);
  if (n > 0) {
    hipLaunchKernelGGL(ref_prep_kernel, dim3(R.G), dim3(kPrepBlock), 0, s, n, means2d, radii, valid, depths, width,
                       height, keys, vals);
    GS_LAUNCH_CHECK("ref_prep_kernel");
    rc = radix_pass<kDepthRB>(s, true, keys, vals, keys2, vals2, nullptr, n, n, 0, R.G, kSpan, table, dtot);
    if (rc != GS_OK) return rc;
    rc = radix_pass<kDepthRB>(s, true, keys2, vals2, keys, vals, nullptr, n, n, kDepthRB, R.G, kSpan, table, dtot);
    if (rc != GS_OK) return rc;
    hipLaunchKernelGGL(ref_sum_kernel, dim3(R.G), dim3(kPrepBlock), 0, s, n, vals, gsum);
    GS_LAUNCH_CHECK("ref_sum_kernel");
    hipLaunchKernelGGL(ref_scan_kernel, dim3(1), dim3(kBig), 0, s, gsum, R.G);
    GS_LAUNCH_CHECK("ref_scan_kernel");
  }
  // with n = 0 gs_bin has cleared the stats and ranges: one workgroup writes the padding
  hipLaunchKernelGGL(ref_fill_kernel, dim3(n > 0 ? R.G : 1), dim3(kPrepBlock), 0, s, n, vals, gsum, stats,
                     R.bin.T, R.L, sorted_tiles, sorted_gids, ranges);
  GS_LAUNCH_CHECK("ref_fill_kernel");
  return GS_OK;
}

// ---------------------------------------------------------------------------------
extern "C" int gs_window_from_bins(void* stream, int64_t n, const float* means2d, const float* radii,
                                   const uint8_t* valid, const float* depths, int width, int height,
                                   const int32_t* sorted_gids, int64_t capacity, const int32_t* stats,
                                   gs_window_t* window) {
  GS_REQUIRE(n >= 0 && n < ((int64_t)1 << 31), "gs_window_from_bins: n must be in [0, 2^31) (got %lld)",
             (long long)n);
  GS_REQUIRE(width > 0 && height > 0, "gs_window_from_bins: bad image size %dx%d", width, height);
  GS_REQUIRE(capacity >= 0 && stats && window, "gs_window_from_bins: bad arguments");
  GS_REQUIRE(n == 0 || (means2d && radii && valid && depths), "gs_window_from_bins: NULL inputs");
  GS_REQUIRE(capacity == 0 || sorted_gids, "gs_window_from_bins: NULL sorted_gids");
  hipLaunchKernelGGL(window_bins_kernel, dim3(1), dim3(kWinThreads), 0, (hipStream_t)stream, n, means2d, radii,
                     valid, depths, width, height, sorted_gids, capacity, stats, window);
  GS_LAUNCH_CHECK("window_bins_kernel");
  return GS_OK;
}
