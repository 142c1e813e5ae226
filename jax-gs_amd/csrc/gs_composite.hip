// Per-tile alpha compositing on gfx950 (forward and backward).
//
// Reference: jax_gs/renderer/rasterizer.py:157-248 (render_tiles): a pixel centre is
// (16*tx + i + 0.5, 16*ty + j + 0.5); the first min(count, 4096) entries of a tile
// are blended front to back; entry k is blended iff T > 1e-4 before it and its
// power > -10, with alpha = min(0.99, exp(power) * sigmoid(opacity)); the pixel is
// C + T * background.  rasterizer_tpu.py computes the same image.
//
// Records hold the conic pre-scaled by log2(e) and log2(sigmoid(opacity)), so one
// exp2 of  q = log2(e) * power + log2(opacity)  gives the unclipped alpha, and the
// gate power > -10 reads  q > log2(opacity) - 10 log2(e)  (a per-entry threshold
// kept in the record).
//
// Work decomposition: every wave owns PPT*4 rows of one 16x16 tile; lane l holds the
// PPT pixels (l % 16, row0 + l / 16 + 4 i), i < PPT, i.e. one column, so the x offset
// to a Gaussian is shared by the lane's pixels.  Waves are independent (no LDS, no
// barriers).  With PPT = 4 a wave covers the whole tile (used for large images);
// PPT = 1 uses four waves per tile for small images that would otherwise leave CUs
// idle; the forward of mid-size images uses PPT = 2 (two waves per tile).
//
// Culling: a Gaussian is binned to every tile its square 3-sigma box touches, but its
// "power > -10" region is an ellipse, and for about a third of the (tile, entry) pairs
// of a dense scene that ellipse reaches no pixel centre of the tile.  Such entries
// change nothing (every pixel gates them out), so a wave first tests 64 entries at a
// time, one per lane, against the rectangle spanned by its pixel centres (exact
// minimum of the convex quadratic form over the rectangle, with a rounding margin,
// so an entry is dropped only if no pixel could pass the gate), and then walks the
// surviving entries.  The walked entry is wave-uniform: its id comes from the
// testing lane and its 48-byte record through scalar loads into SGPRs, prefetched
// one surviving entry ahead.
//
// Forward: branch-free per pixel; the wave stops when every pixel has T <= 1e-4
// (ballot every 8 walked entries).  Per pixel it writes the final T and n_contrib,
// the number of leading entries met while T > 1e-4 (culled entries included).
// Backward: replays each pixel back to front from (final T, n_contrib), recovering
// T_k = T_{k+1} / (1 - alpha_k) and the colour behind entry k projected on the
// pixel's image cotangent g, Rg_{k-1} = alpha_k (c_k . g) + (1 - alpha_k) Rg_k, so
// dL/dalpha_k = T_k (c_k . g - Rg_k).  Per lane the entry's power cotangents are kept
// as sums that the lane's pixels (one column, one dx) share; the 9 sums of four
// walked entries are reduce-scattered across the wave together (recursive halving, so
// each of 36 lanes ends with the total of one sum) and added to the Gaussians' gradient
// records with one atomic instruction (36 lanes).  Gradients follow JAX autodiff of the
// reference: the cap
// min(0.99, .) passes no gradient when it binds (half at a tie), gated entries pass
// none.
#include "gs_bins.h"
#include "gs_common.h"
#include "gs_cull.h"

#include <algorithm>

namespace gs {
namespace {

constexpr float kTMin = 1e-4f;
// s_waitcnt immediate (gfx9 layout) that waits for lgkmcnt = 0 and for nothing else
constexpr int kWaitLgkm0 = 0xC07F;

__device__ inline float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ inline int bcast_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

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

// The image cotangent the backward reads per pixel: dL/dimage (gimg), and/or the VJP of the
// L1 loss fused into the compositing (losses.py:4-8) when tgt is set: sign(image - target)
// times (dL/dloss) / count, sign(0) = 0, formed as the separate loss VJP forms it.
struct ImageCot {
  const float* gimg;  // may be NULL when tgt is set
  const float* img;   // the forward's image (fused L1)
  const float* tgt;   // L1 target; NULL: no fused L1
  const float* cot;   // dL/dloss, one float on the device
};
__device__ inline float l1_sign(float d) { return d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f); }
__device__ inline float l1_scale(const ImageCot& c, int W, int H) {
  return c.tgt != nullptr ? c.cot[0] / (float)(3 * (int64_t)W * H) : 0.0f;
}
__device__ inline void image_cot(const ImageCot& c, float sc, int64_t p, float& g0, float& g1, float& g2) {
  if (c.tgt == nullptr) {
    g0 = c.gimg[3 * p];
    g1 = c.gimg[3 * p + 1];
    g2 = c.gimg[3 * p + 2];
    return;
  }
  g0 = l1_sign(c.img[3 * p] - c.tgt[3 * p]) * sc;
  g1 = l1_sign(c.img[3 * p + 1] - c.tgt[3 * p + 1]) * sc;
  g2 = l1_sign(c.img[3 * p + 2] - c.tgt[3 * p + 2]) * sc;
  if (c.gimg != nullptr) {
    g0 += c.gimg[3 * p];
    g1 += c.gimg[3 * p + 1];
    g2 += c.gimg[3 * p + 2];
  }
}

// Reduce-scatter of per-lane values over the wave by recursive halving.  A level pairs
// the values (2k, 2k+1); a lane keeps the member selected by one of its lane bits and
// adds the partner lane's copy of it (partner = lane ^ distance).  The levels run in
// the order of lane distance 32, 16, 8, 4, 2, so the wide levels (many values) use the
// two-instruction forms:
//   32, 16: v_permlane32_swap / v_permlane16_swap exchange the upper half of the low
//           value with the lower half of the high value, after which every lane adds
//           its two registers;
//   8, 4:   two DPP adds restricted by bank masks (banks = groups of 4 lanes of a
//           16-lane row): the lanes with a clear distance bit add the low value of
//           lane + d into their low register, then the others add the high value of
//           lane - d into the same register;
//   2:      select the kept and the sent value and add the partner's (quad_perm DPP).
// The last level (distance 1) is a plain pairwise sum, so lanes l and l ^ 1 end with the
// same total.
__device__ inline float add_swap32(float lo, float hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float add_swap16(float lo, float hi) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The DPP adds are inline assembly (a masked DPP add that keeps the other lanes'
// destination has no builtin form).  Each starts with two wait states: a VALU write of
// a VGPR followed by a DPP read of it needs them, and the compiler's hazard checks do
// not look inside inline assembly.
#define GS_DPP_ADD_SELF(dst, ctrl, banks) \
  asm volatile("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 " ctrl " row_mask:0xf bank_mask:" banks : "+v"(dst))
#define GS_DPP_ADD(dst, src, ctrl, banks) \
  asm volatile("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 " ctrl " row_mask:0xf bank_mask:" banks : "+v"(dst) : "v"(src))

template <int D>
__device__ inline float add_banked(float lo, float hi, bool has_hi) {
  if (D == 8) {
    GS_DPP_ADD_SELF(lo, "row_shl:8", "0x3");
    if (has_hi) GS_DPP_ADD(lo, hi, "row_shr:8", "0xc");
  } else {
    GS_DPP_ADD_SELF(lo, "row_shl:4", "0x5");
    if (has_hi) GS_DPP_ADD(lo, hi, "row_shr:4", "0xa");
  }
  return lo;
}
#undef GS_DPP_ADD
#undef GS_DPP_ADD_SELF

template <int D, int N>
__device__ inline void halve_level(float* cur, int lane) {
#pragma unroll
  for (int k = 0; k < (N + 1) / 2; ++k) {
    const bool has_hi = 2 * k + 1 < N;
    const float lo = cur[2 * k];
    const float hi = has_hi ? cur[2 * k + 1] : lo;  // a missing high value: its slot is never read
    if (D == 32) {
      cur[k] = add_swap32(lo, hi);
    } else if (D == 16) {
      cur[k] = add_swap16(lo, hi);
    } else if (D == 8 || D == 4) {
      cur[k] = add_banked<D>(lo, hi, has_hi);
    } else if (D == 2) {
      const bool bit = (lane >> 1) & 1;
      const float keep = bit ? hi : lo, send = bit ? lo : hi;
      cur[k] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x4E, 0xF, 0xF, false));
    } else {  // D == 1
      const bool bit = lane & 1;
      const float keep = bit ? hi : lo, send = bit ? lo : hi;
      cur[k] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0xB1, 0xF, 0xF, false));
    }
  }
}

// The backward's reduce-scatter of four walked entries.  Per entry a lane holds six sums
// over its pixels, (P, Q, V, c0, c1, c2) = sum dpower, sum dpower dy, sum dpower dy^2 and
// the colour cotangents, all for its own column dx = px - mean.x.  The first level runs per
// pair of entries as soon as the pair is walked (lane bit 5 keeps entry 0 of the pair, else
// entry 1), so only one pair's twelve sums are live at a time; the second (distance 16)
// keeps pair 0 where lane bit 4 is clear.  Lanes l, l ^ 16, l ^ 32 and l ^ 48 share
// the column, so after these two levels each lane holds the column sums of entry
// quad_entry(l) = 2 bit4 + bit5; it expands them into the record's nine values and the
// levels 8 .. 1 reduce-scatter those over the 16 lanes of the entry: lane l ends with the
// total of record value quad9_index(l) (bit-reversed low four bits; 9 .. 15 hold nothing).
// Per entry this takes about 16 VALU instructions against about 22 for two entries at a
// time.
__device__ inline int quad_entry(int l) { return ((l >> 3) & 2) | ((l >> 5) & 1); }
__device__ inline int quad9_index(int l) { return ((l & 1) << 3) | ((l & 2) << 1) | ((l >> 1) & 2) | ((l >> 3) & 1); }

__device__ inline void pair_level32(const float* sa, const float* sb, float* out) {
  float cur[12];
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    cur[2 * k] = sa[k];
    cur[2 * k + 1] = sb[k];
  }
  halve_level<32, 12>(cur, 0);
#pragma unroll
  for (int k = 0; k < 6; ++k) out[k] = cur[k];
}

__device__ inline float reduce_scatter_quad9(const float* p0, const float* p1, float dx0, float dx1, float dx2,
                                             float dx3, int lane) {
  float cur[12];
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    cur[2 * k] = p0[k];
    cur[2 * k + 1] = p1[k];
  }
  halve_level<16, 12>(cur, lane);
  const bool b4 = (lane >> 4) & 1, b5 = (lane >> 5) & 1;
  const float dx01 = b5 ? dx1 : dx0, dx23 = b5 ? dx3 : dx2;
  const float dx = b4 ? dx23 : dx01;
  const float Sx = cur[0] * dx;
  float v[9] = {Sx, cur[1], Sx * dx, cur[1] * dx, cur[2], cur[0], cur[3], cur[4], cur[5]};
  halve_level<8, 9>(v, lane);
  halve_level<4, 5>(v, lane);
  halve_level<2, 3>(v, lane);
  halve_level<1, 2>(v, lane);
  return v[0];
}

// XCD-aware tile order. Consecutive workgroups go round-robin to the 8 XCDs. The tile grid,
// padded to a multiple of 8 x 4 tiles, is cut into cells of 2 x 2 tiles; XCD x = b % 8 takes
// the cells whose column is x % 4 and whose row is x / 4 modulo (4, 2). Every XCD thus holds
// an even sample of the image, so its share of the work does not depend on where the
// scene's content lies (contiguous bands of rows gave the busiest XCD 1.23x the mean on a
// centred scene), while the four tiles of a cell, which share most of their Gaussians, hit
// one L2. A cell's tiles go to consecutive workgroups of the XCD, i.e. to different SIMDs.
// This holds for one wave per tile.  With WPT waves per tile the kernels take
// b = blockIdx.x / WPT, so a tile's waves are consecutive workgroups on WPT different XCDs
// and each of those L2s fetches the tile's records; keeping a tile's waves on one XCD was
// measured no faster (those launches are latency-bound, not L2-bound).
__host__ __device__ inline int tile_blocks(int TX, int TY) { return ((TX + 7) & ~7) * ((TY + 3) & ~3); }

// Tile of workgroup b (b < tile_blocks(TX, TY)), or -1 for a padding workgroup.
__device__ inline int tile_of_block(int b, int TX, int TY) {
  const int U = (TX + 7) >> 3;
  const int x = b & 7, j = b >> 3, k = j >> 2;
  const int tx = 8 * (k % U) + 2 * (x & 3) + (j & 1);
  const int ty = 4 * (k / U) + 2 * (x >> 2) + ((j >> 1) & 1);
  return (tx < TX && ty < TY) ? ty * TX + tx : -1;
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

// One compositing record (layout of GS_REC_STRIDE floats in gs_raster.h).
struct Rec {
  float mx, my, A, B, C, lop, r, g, b, op, thr, no_cap;
};

__device__ inline Rec zero_rec() { return Rec{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}; }

__device__ inline Rec load_rec(const float4* __restrict__ rec, int g) {
  const float4 a = rec[(int64_t)g * 3];
  const float4 b = rec[(int64_t)g * 3 + 1];
  const float4 c = rec[(int64_t)g * 3 + 2];
  return Rec{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w};
}

// A walked entry's record is addressed by a value read from the testing lane: with O32
// the byte offset gid * 48 (records below 4 GiB), which scalar loads take as their
// offset register (one lane read and the loads, no 64-bit address arithmetic per entry);
// otherwise the id.  The gradient records have the same 48-byte stride.
template <bool O32>
__device__ inline int rec_key(int g) { return O32 ? (int)((uint32_t)g * (uint32_t)(kRec * 4)) : g; }

template <bool O32>
__device__ inline Rec load_rec_key(const float4* __restrict__ rec, int key) {
  if (!O32) return load_rec(rec, key);
  const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const char*>(rec) + (uint32_t)key);
  const float4 a = p[0], b = p[1], c = p[2];
  return Rec{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w};
}

template <bool O32>
__device__ inline float* grec_at(float* __restrict__ grec, int key, int v) {
  return O32 ? reinterpret_cast<float*>(reinterpret_cast<char*>(grec) + (uint32_t)key) + v
             : grec + (int64_t)key * kRec + v;
}

// Ids are clamped like XLA's gather.
__device__ inline int clamp_gid(int g, int num_g) { return min(max(g, 0), num_g - 1); }

// What a lane fetches to test one entry of a batch against the wave's pixel
// rectangle: the (clamped) id, or -1 past the tile's list, and the record's centre
// and conic.  Batches are software-pipelined: the ids of batch b+2 and the records of
// batch b+1 are in flight while batch b is walked.
struct Probe {
  int g;
  float mx, my, A, B, C;
};

// Id of entry k of a tile whose entries start at `start` (-1 past the n entries).
// Without a window: the tile's own entries (rasterizer_tpu.py:90-97 gathers them one by
// one).  With one (WIN): the default path's chunk windows (rasterizer.py:184-190): chunk
// c = k / 512 slices 512 ids at min(start + 512 c, L - 512) of the reference's L-slot
// arrays, so a chunk that starts past thr = L - 512 (in this list's coordinates) reads the
// arrays' last 512 slots, held in win->ids.  The test is uniform over a batch of 64.
template <bool WIN>
__device__ inline int probe_gid(const int32_t* __restrict__ gids, int start, int k, int n, int num_g,
                                const gs_window_t* __restrict__ win, int64_t thr) {
  if (k < 0 || k >= n) return -1;
  const int32_t* src = gids + ((int64_t)start + k);
  if (WIN && (int64_t)start + (k & ~(kBlock - 1)) > thr) src = win->ids + (k & (kBlock - 1));
  return clamp_gid(*src, num_g);
}

// The same split in two: the load of a batch ahead (raw id, and whether k is an entry),
// and the clamp where the id is used, a batch later, so that nothing waits for the load
// in between (a clamp right after it waits for every load in flight).  Both walks use it
// (backward cfg2 311 -> 307 us).
struct Ahead {
  int raw;
  bool ok;
};
template <bool WIN>
__device__ inline Ahead probe_gid_ahead(const int32_t* __restrict__ gids, int start, int k, int n,
                                        const gs_window_t* __restrict__ win, int64_t thr) {
  Ahead a{0, k >= 0 && k < n};
  if (a.ok) {
    const int32_t* src = gids + ((int64_t)start + k);
    if (WIN && (int64_t)start + (k & ~(kBlock - 1)) > thr) src = win->ids + (k & (kBlock - 1));
    a.raw = *src;
  }
  return a;
}
__device__ inline int ahead_gid(const Ahead& a, int num_g) { return a.ok ? clamp_gid(a.raw, num_g) : -1; }

__device__ inline Probe probe_load(const float4* __restrict__ rec, int g) {
  Probe p{g, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  if (g >= 0) {
    const float4 a = rec[(int64_t)g * 3];
    p.mx = a.x;
    p.my = a.y;
    p.A = a.z;
    p.B = a.w;
    p.C = rec[(int64_t)g * 3 + 1].x;
  }
  return p;
}

// Ballot of the entries of a batch that survive the rectangle test.
__device__ inline uint64_t probe_test(const Probe& p, float x0, float x1, float y0, float y1) {
  return __ballot(p.g >= 0 && !entry_misses_rect(p.mx, p.my, p.A, p.B, p.C, x0, x1, y0, y1));
}

// WIN: the default path's chunk windows (see probe_gid); without it the id fetch compiles
// to the plain one.
// SB (gs_composite_fwd_deferred): when the binning deferred the entry list
// (entries_deferred), each wave takes its tile's entries from its superblock's list
// (gs_bins.h): the words whose bit is set in the tile's step masks, in the list's order.
// It writes the ids of the entries it probes to gids_out[start + k] (whole batches, so every
// entry below the tile's largest n_contrib -- the part of the list the backward replays --
// is written) and stops where the walk over the entry list would stop.  Otherwise it walks
// the entry list as without SB.
template <int PPT, bool WIN, bool O32, bool SB>
__global__ __launch_bounds__(64) void composite_fwd_kernel(
    const float4* __restrict__ rec, int num_g, const int32_t* __restrict__ gids, int64_t n_entries,
    const int32_t* __restrict__ ranges, int W, int H, int TX, int T, const float* __restrict__ bg,
    float* __restrict__ img, float* __restrict__ finalT, int32_t* __restrict__ ncontrib,
    int32_t* __restrict__ tile_cost, float4* __restrict__ clear, int64_t n_clear,
    const gs_window_t* __restrict__ win, const SBLists sbl, int32_t* __restrict__ gids_out,
    const float* __restrict__ l1_tgt, float* __restrict__ l1_part) {
  constexpr int WPT = 4 / PPT;  // waves per tile
  // Every workgroup clears its slice of the caller's array after its own outputs (stores
  // and loads share one wait counter, so stores issued before the walk would hold up its
  // first loads).
  auto clear_slice = [&]() {
    if (clear != nullptr) {
      const int64_t per = (n_clear + gridDim.x - 1) / gridDim.x;
      const int64_t c0 = per * blockIdx.x, c1 = c0 + per < n_clear ? c0 + per : n_clear;
      for (int64_t c = c0 + threadIdx.x; c < c1; c += 64) clear[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  const int b = blockIdx.x / WPT, part = blockIdx.x % WPT;
  const int tile = tile_of_block(b, TX, T / TX);
  if (tile < 0) {
    if (l1_part != nullptr && threadIdx.x == 0) l1_part[blockIdx.x] = 0.0f;
    clear_slice();
    return;
  }
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
  const float rx0 = (float)(tx * kTile) + 0.5f, rx1 = rx0 + (float)(kTile - 1);
  const float ry0 = (float)(ty * kTile + part * 4 * PPT) + 0.5f, ry1 = ry0 + (float)(4 * PPT - 1);

  bool done = false;
  int walked = 0;
  // Walks the survivors m of a batch (lane j's record key in gk); kpos(j) is the index in
  // the tile's list of the batch's entry j.
  auto walk = [&](uint64_t m, const int gk, auto kpos) {
    // Survivors are walked in groups of G (G = 2 when a lane holds one pixel): the
    // group's records are in SGPRs before it is blended and the next group's scalar
    // loads are issued first, so their latency is covered by G entries' arithmetic
    // (scalar loads complete out of order: waiting for one is waiting for all, so
    // requests go out per group).  With two or four pixels per lane the arithmetic of one
    // entry covers the load and G = 1 keeps the instruction count down; its two record
    // registers are used in turn, with an explicit wait before each request (two-wave
    // forward, cfg4 175 -> 155 us, cfg3 148 -> 135 us; one-wave cfg2 unchanged).
    constexpr int G = PPT == 1 ? 2 : 1;
    // one walked entry e (tile index kidx within the batch) blended into the lane's pixels
    // (two or four pixels per lane: branch-free, gated-out pixels blend alpha = 0, which
    // leaves C and T unchanged; measured faster than per-pixel branches, 226 vs 251 us
    // on cfg2)
    auto blend = [&](const Rec& e, int kidx) {
      const int kk = kpos(kidx) + 1;  // entries met so far, this one included
      const float dx = px - e.mx;
      const float Adx2l = fmaf(e.A * dx, dx, e.lop), Bdx = e.B * dx;
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const float q = q_of(py[i] - e.my, Adx2l, Bdx, e.C);
        const bool act = Tr[i] > kTMin;  // rasterizer.py:206
        float al = __builtin_amdgcn_exp2f(q);
        al = al < 0.99f ? al : 0.99f;
        al = (act && q > e.thr) ? al : 0.0f;  // rasterizer.py:212
        const float w = al * Tr[i];
        c0[i] = fmaf(w, e.r, c0[i]);
        c1[i] = fmaf(w, e.g, c1[i]);
        c2[i] = fmaf(w, e.b, c2[i]);
        Tr[i] = Tr[i] - w;  // T (1 - alpha)
        cnt[i] = act ? kk : cnt[i];
      }
    };
    if constexpr (G == 1) {
      // one entry at a time, the next survivor's record requested before the blend; two
      // record registers used in turn (no copy of the prefetched record per entry)
      Rec ra = zero_rec(), rb = zero_rec();
      int ja = -1, jb = -1;
      if (m != 0ull) {
        ja = __builtin_ctzll(m);
        m &= ~(1ull << ja);
        ra = load_rec_key<O32>(rec, bcast_i(gk, ja));
      }
      // survivors in groups of 8 (four rounds of the two registers), the wave's exit test
      // once per group: no per-entry bookkeeping for it
      bool more = ja >= 0;
      while (more) {
        bool live = false;
#pragma unroll
        for (int i = 0; i < PPT; ++i) live = live || Tr[i] > kTMin;
        if (__ballot(live) == 0ull) {
          done = true;
          break;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          // ra's record was requested a whole entry ago: wait for it before the next
          // request goes out (scalar loads complete out of order, so a wait at its first
          // use would also wait for the request issued just before)
          __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
          jb = -1;
          if (m != 0ull) {
            jb = __builtin_ctzll(m);
            m &= ~(1ull << jb);
            rb = load_rec_key<O32>(rec, bcast_i(gk, jb));
          }
          ++walked;
          blend(ra, ja);
          if (jb < 0) {
            more = false;
            break;
          }
          __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
          ja = -1;
          if (m != 0ull) {
            ja = __builtin_ctzll(m);
            m &= ~(1ull << ja);
            ra = load_rec_key<O32>(rec, bcast_i(gk, ja));
          }
          ++walked;
          blend(rb, jb);
          if (ja < 0) {
            more = false;
            break;
          }
        }
      }
    } else {
      // one pixel per lane: survivors in pairs, both records requested together a pair
      // ahead, two pairs of record registers used in turn, the exit test once per 8
      auto take = [&](Rec* r, int* j) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
          j[h] = -1;
          if (m != 0ull) {
            j[h] = __builtin_ctzll(m);
            m &= ~(1ull << j[h]);
            r[h] = load_rec_key<O32>(rec, bcast_i(gk, j[h]));
          }
        }
      };
      auto blend_pair = [&](const Rec* e, const int* k) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
          if (k[h] < 0) break;
          ++walked;
          const int kk = kpos(k[h]) + 1;  // entries met so far, this one included
          const float dx = px - e[h].mx;
          const float Adx2l = fmaf(e[h].A * dx, dx, e[h].lop), Bdx = e[h].B * dx;
#pragma unroll
          for (int i = 0; i < PPT; ++i) {
            const float q = q_of(py[i] - e[h].my, Adx2l, Bdx, e[h].C);
            const bool act = Tr[i] > kTMin;  // rasterizer.py:206
            cnt[i] = act ? kk : cnt[i];
            // one pixel per lane: only the lanes that pass run the blend (the wave skips it
            // when none does; cfg1 187 -> 180 us against the branch-free form)
            if (act && q > e[h].thr) {  // rasterizer.py:212
              float al = __builtin_amdgcn_exp2f(q);
              al = al < 0.99f ? al : 0.99f;
              const float w = al * Tr[i];
              c0[i] = fmaf(w, e[h].r, c0[i]);
              c1[i] = fmaf(w, e[h].g, c1[i]);
              c2[i] = fmaf(w, e[h].b, c2[i]);
              Tr[i] = Tr[i] - w;  // T (1 - alpha)
            }
          }
        }
      };
      Rec ra[G], rb[G];
      int ja[G], jb[G];
#pragma unroll
      for (int h = 0; h < G; ++h) ra[h] = rb[h] = zero_rec();
      take(ra, ja);
      bool more = ja[0] >= 0;
      while (more) {
        bool live = false;
#pragma unroll
        for (int i = 0; i < PPT; ++i) live = live || Tr[i] > kTMin;
        if (__ballot(live) == 0ull) {
          done = true;
          break;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
          take(rb, jb);
          blend_pair(ra, ja);
          if (jb[0] < 0) {
            more = false;
            break;
          }
          __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
          take(ra, ja);
          blend_pair(rb, jb);
          if (ja[0] < 0) {
            more = false;
            break;
          }
        }
      }
    }
  };

  bool deferred = false;
  if constexpr (SB) deferred = entries_deferred(sbl.stats);
  if (!deferred) {
    const int64_t thr = WIN ? win->thr : 0;
    // The batch's probe records were requested a batch ago; the next batch's go out after
    // the batch's test, so that the test waits for nothing requested since (loads complete
    // in order: a wait for one waits for every earlier one), and the id two batches ahead
    // is clamped where it is used, a batch later.
    Ahead g_ahead = probe_gid_ahead<WIN>(gids, start, 64 + lane, n, win, thr);
    Probe pr = probe_load(rec, probe_gid<WIN>(gids, start, lane, n, num_g, win, thr));
    for (int b0 = 0; b0 < n && !done; b0 += 64) {
      const int gk = rec_key<O32>(pr.g);  // the lane's record key (read where the lane survives)
      const uint64_t m = probe_test(pr, rx0, rx1, ry0, ry1);
      pr = probe_load(rec, ahead_gid(g_ahead, num_g));
      g_ahead = probe_gid_ahead<WIN>(gids, start, b0 + 128 + lane, n, win, thr);
      walk(m, gk, [&](int j) { return b0 + j; });
    }
  } else if constexpr (SB) {
    if (n > 0) {
      // The tile's entries, in order, are the words of its superblock's list whose bit is set
      // in the tile's step masks (the binning's count sweep wrote them).  A ring of 512 word
      // positions in LDS queues the entries, so that they are probed and walked in full
      // batches of 64 as above: fill(t) queues entries until t are queued (or the list ends),
      // one chunk (four steps of 64 words, one mask each) at a time.  The masks of 16 chunks (64 steps) come with
      // one vector load (lane l: step l), the next 16 a group ahead.  Entry k's id is written
      // to gids_out[start + k] when its batch is probed (the backward's list).
      constexpr int kRing = 512;  // live entries span < 64 + 256 (a fill overshoots by < 4 steps)
      __shared__ int32_t q_lds[kRing];
      volatile int32_t* q = q_lds;  // lanes read what other lanes wrote: keep the order
      const int sx = tx / kSB, sy = ty / kSB;
      const int sbi = sy * sbl.SX + sx;
      const int u = (ty - sy * kSB) * kSB + (tx - sx * kSB);
      int64_t c0 = sbl.chunk_base[sbi], c1 = sbl.chunk_base[sbi + 1];
      c0 = c0 > sbl.n_chunks ? sbl.n_chunks : c0;
      c1 = c1 < c0 ? c0 : (c1 > sbl.n_chunks ? sbl.n_chunks : c1);
      const int64_t wbase = sbl.ranges[sbi];
      const int nsteps = 4 * (int)(c1 - c0);
      auto group = [&](int gi) -> uint64_t {
        const int64_t c = c0 + 16 * (int64_t)gi + (lane >> 2);
        return c < c1 ? sbl.masks[(c * 64 + u) * 4 + (lane & 3)] : 0ull;
      };
      uint64_t mg = group(0), mg_next = group(1);
      int sidx = 0, filled = 0;
      // a chunk (four steps) per round: its eight mask halves are read together
      auto fill = [&](int target) {
        while (filled < target && sidx < nsteps) {
          if (sidx > 0 && (sidx & 63) == 0) {
            mg = mg_next;
            mg_next = group((sidx >> 6) + 1);
          }
          uint32_t lo[4], hi[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            lo[k] = __builtin_amdgcn_readlane((uint32_t)mg, (sidx & 63) + k);
            hi[k] = __builtin_amdgcn_readlane((uint32_t)(mg >> 32), (sidx & 63) + k);
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint64_t m = ((uint64_t)hi[k] << 32) | lo[k];
            if (m != 0ull) {
              if (__builtin_amdgcn_inverse_ballot_w64(m))
                q[(filled + (int)__builtin_amdgcn_mbcnt_hi(hi[k], __builtin_amdgcn_mbcnt_lo(lo[k], 0u))) &
                  (kRing - 1)] = (int32_t)(wbase + 64 * (int64_t)(sidx + k) + lane);
              filled += __popcll(m);
            }
          }
          sidx += 4;
        }
      };
      // entry k's word (its low half, which holds the id; loaded a batch ahead of its use),
      // none past the queued entries
      struct WordAhead {
        uint32_t w;
        bool ok;
      };
      const uint32_t* __restrict__ word_lo = reinterpret_cast<const uint32_t*>(sbl.words);
      auto word_ahead = [&](int k) {
        WordAhead a{0u, k < n && k < filled};
        if (a.ok) {
          const int64_t pos = q[k & (kRing - 1)];
          a.ok = pos >= 0 && pos < sbl.n_words;
          if (a.ok) a.w = word_lo[2 * pos];
        }
        return a;
      };
      // the id where it is used, a batch later; stored for the backward
      auto take_gid = [&](const WordAhead& a, int k) {
        if (!a.ok) return -1;
        const int g = clamp_gid((int)(a.w & 0x3FFFFFFu), num_g);
        gids_out[start + k] = g;  // k < n: inside the tile's range
        return g;
      };
      fill(128);
      WordAhead a_ahead = word_ahead(64 + lane);
      Probe pr = probe_load(rec, take_gid(word_ahead(lane), lane));
      for (int b0 = 0; b0 < n && !done; b0 += 64) {
        const int gk = rec_key<O32>(pr.g);
        const uint64_t m = probe_test(pr, rx0, rx1, ry0, ry1);
        pr = probe_load(rec, take_gid(a_ahead, b0 + 64 + lane));
        fill(b0 + 192);
        a_ahead = word_ahead(b0 + 128 + lane);
        walk(m, gk, [&](int j) { return b0 + j; });
      }
    }
  }
  const float bg0 = bg[0], bg1 = bg[1], bg2 = bg[2];
  // the L1 loss against l1_tgt (losses.py:4-8): the lane's sum of |image - target| over its
  // pixels' channels, reduced over the wave into the workgroup's partial
  float l1 = 0.0f;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int Y = Y0 + 4 * i;
    if (X < W && Y < H) {
      const int64_t p = (int64_t)Y * W + X;
      const float o0 = c0[i] + Tr[i] * bg0, o1 = c1[i] + Tr[i] * bg1, o2 = c2[i] + Tr[i] * bg2;
      img[3 * p] = o0;
      img[3 * p + 1] = o1;
      img[3 * p + 2] = o2;
      if (finalT) finalT[p] = Tr[i];
      // a pixel still open met every entry of the tile, culled ones included
      if (ncontrib) ncontrib[p] = Tr[i] > kTMin ? n : cnt[i];
      if (l1_tgt != nullptr)
        l1 += (fabsf(o0 - l1_tgt[3 * p]) + fabsf(o1 - l1_tgt[3 * p + 1])) + fabsf(o2 - l1_tgt[3 * p + 2]);
    }
  }
  if (l1_part != nullptr) {
    l1 = wave_sum(l1);
    if (lane == 0) l1_part[blockIdx.x] = l1;
  }
  // walk length of the tile (first wave of the tile): the backward's cost estimate
  // (two waves per tile: each stores its own length in one 16-bit half, the order takes
  // the longer; lengths are at most kMaxTileEntries)
  if (tile_cost && lane == 0) {
    if (WPT == 2)
      reinterpret_cast<uint16_t*>(tile_cost)[2 * tile + part] = (uint16_t)walked;
    else if (part == 0)
      tile_cost[tile] = walked;
  }
  clear_slice();
}

// NOCAP: the body without the cap's per-pixel selections (the cap is applied to the alphas
// in place, and the power sums redone with its selections, only for entries that some pixel
// of the wave can see at the cap), with 1/T as the per-pixel state: T_k = 1/(1/T_{k+1} *
// (1 - alpha_k)) costs an fma and an rcp where T_{k+1}/(1 - alpha_k) costs a subtraction,
// an rcp and a product.  Both NOCAP changes keep the loop-carried state in place (a body
// chosen per entry between two versions made the compiler copy that state at every entry).
// More registers live than the 64-VGPR build allows.
template <int PPT, bool WIN, bool NOCAP, bool O32>
__device__ __forceinline__ void composite_bwd_body(
    const float4* __restrict__ rec, int num_g, const int32_t* __restrict__ gids, int64_t n_entries,
    const int32_t* __restrict__ ranges, int W, int H, int TX, int T, const float* __restrict__ bg,
    const ImageCot gc, const float* __restrict__ finalT, const int32_t* __restrict__ ncontrib,
    float* __restrict__ grec, const int32_t* __restrict__ order, const gs_window_t* __restrict__ win) {
  constexpr int WPT = 4 / PPT;
  const int b = blockIdx.x / WPT, part = blockIdx.x % WPT;
  const int tile = order ? (b < T ? order[b] : -1) : tile_of_block(b, TX, T / TX);
  if (tile < 0 || tile >= T) return;
  const int lane = threadIdx.x;
  const int tx = tile % TX, ty = tile / TX;
  const int X = tx * kTile + (lane & 15);
  const int Y0 = ty * kTile + part * 4 * PPT + (lane >> 4);
  const float px = (float)(tx * kTile) + ((float)(lane & 15) + 0.5f);
  int start, n;
  tile_span(ranges, tile, n_entries, num_g, start, n);
  const float bg0 = bg[0], bg1 = bg[1], bg2 = bg[2];
  const float l1sc = l1_scale(gc, W, H);

  float py[PPT], Tr[PPT], g0[PPT], g1[PPT], g2[PPT], Rg[PPT];
  int kp[PPT];
  int kmax = 0, kmin = 1 << 30;
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int yl = part * 4 * PPT + (lane >> 4) + 4 * i;
    py[i] = (float)(ty * kTile) + ((float)yl + 0.5f);
    Tr[i] = 1.0f;  // NOCAP: the reciprocal 1/T (see the body)
    g0[i] = g1[i] = g2[i] = 0.0f;
    kp[i] = 0;
    const int Y = Y0 + 4 * i;
    if (X < W && Y < H) {
      const int64_t p = (int64_t)Y * W + X;
      Tr[i] = NOCAP ? 1.0f / fmaxf(finalT[p], 1e-30f) : finalT[p];  // finite for T = 0
      const int k = ncontrib[p];
      kp[i] = k < 0 ? 0 : (k > n ? n : k);  // entries beyond the tile's list never load
      image_cot(gc, l1sc, p, g0[i], g1[i], g2[i]);
    }
    // colour behind the last entry is the background
    Rg[i] = fmaf(bg2, g2[i], fmaf(bg1, g1[i], bg0 * g0[i]));
    kmax = max(kmax, kp[i]);
    kmin = min(kmin, X < W && Y0 + 4 * i < H ? kp[i] : 0);
  }
  // wave-wide maximum entry count (uniform loop bound); the wave-wide minimum: below it
  // every pixel of the wave is inside the image and still open (k < kp)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    kmax = max(kmax, __shfl_xor(kmax, o, 64));
    kmin = min(kmin, __shfl_xor(kmin, o, 64));
  }
  kmax = bcast_i(kmax, 0);
  kmin = bcast_i(kmin, 0);

  // entries kmax-1 .. 0 in batches of 64 from the top; surviving entries walked from
  // the highest down, ids from the testing lane, records by scalar loads, prefetched
  const float rx0 = (float)(tx * kTile) + 0.5f, rx1 = rx0 + (float)(kTile - 1);
  const float ry0 = (float)(ty * kTile + part * 4 * PPT) + 0.5f, ry1 = ry0 + (float)(4 * PPT - 1);
  // survivors are walked four at a time and their sums reduced together (one
  // reduce-scatter of several entries' sums costs fewer cross-lane steps per entry than
  // one per entry)
  const int btop = (kmax - 1) & ~63;
  const int64_t thr = WIN ? win->thr : 0;
  Ahead g_ahead = probe_gid_ahead<WIN>(gids, start, btop - 64 + lane, kmax, win, thr);
  Probe p_next = probe_load(rec, probe_gid<WIN>(gids, start, btop + lane, kmax, num_g, win, thr));
  for (int b0 = btop; b0 >= 0; b0 -= 64) {
    const Probe pr = p_next;
    p_next = probe_load(rec, ahead_gid(g_ahead, num_g));
    g_ahead = probe_gid_ahead<WIN>(gids, start, b0 - 128 + lane, kmax, win, thr);
    const int gk = rec_key<O32>(pr.g);  // the lane's record key (read where the lane survives)
    // KT: whether the walk tests k < kp per pixel; the no-cap body drops the test for a
    // batch whose entries all lie below every pixel's count (most batches of a tile).  The
    // survivor mask and the prefetch state are the walk's own (captured by reference, the
    // one-pixel build kept wave-uniform values in vector registers: cfg1 211 -> 226 us).
    auto walk = [&](auto kt_tag, uint64_t m) {
    constexpr bool KT = decltype(kt_tag)::value;
    // the next survivor's record is requested one entry ahead, into ra for the first
    // half of a pair and rb for the second (used in turn: no copy per entry)
    Rec ra = zero_rec(), rb = zero_rec();
    int jn = 0, gn = 0;
    if (m != 0ull) {
      jn = 63 - __builtin_clzll(m);
      gn = bcast_i(gk, jn);
      ra = load_rec_key<O32>(rec, gn);
    }
    while (m != 0ull) {
      constexpr int E = 4;  // walked entries per reduce-scatter
      float s6[E][6], dxh[E], p0[6];
      bool any = false;
      int gh[E];
#pragma unroll
      for (int h = 0; h < E; ++h) {
        // h > 0 with no survivor left: an empty entry (all sums 0); the first always has
        // one (the loop's condition)
        const Rec& e = (h & 1) == 0 ? ra : rb;
        Rec& ahead = (h & 1) == 0 ? rb : ra;
        const int g = gn;
        const bool live = h == 0 || m != 0ull;
        const int k = b0 + jn;
        if (live) {
          // e was requested an entry ago: wait for it before the next request goes out
          // (scalar loads complete out of order)
          __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
          m &= ~(1ull << jn);
          if (m != 0ull) {
            jn = 63 - __builtin_clzll(m);
            gn = bcast_i(gk, jn);
            ahead = load_rec_key<O32>(rec, gn);
          }
        }
        gh[h] = (h == 0 || live) ? g : gh[0];
        const float dx = px - e.mx;
        const float Adx2l = fmaf(e.A * dx, dx, e.lop), Bdx = e.B * dx;
        // per-lane sums over the lane's pixels: P = sum dpower, Q = sum dpower*dy,
        // V = sum dpower*dy^2, colour cotangents (from -0, so that the first term is
        // the sum itself)
        float P = -0.0f, Q = -0.0f, V = -0.0f, gc0 = -0.0f, gc1 = -0.0f, gc2 = -0.0f;
        if (live) {
        float dyv[PPT], qv[PPT];
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
          dyv[i] = py[i] - e.my;
          qv[i] = q_of(dyv[i], Adx2l, Bdx, e.C);
        }
        if (NOCAP) {
          // alpha of each pixel, capped only when some pixel of the wave can reach the
          // 0.99 cap with this entry (rare): below it min(araw, 0.99) = araw, and the
          // cotangent passes whole, so the body needs no selections; the rare capped
          // entry redoes its power sums with the cap's selections afterwards.  One body
          // for both keeps the per-pixel state (T, Rg) in place across entries.
          // (the record's flag first: most records provably cannot reach the cap at all;
          // only the exact value 1.0 skips the test, so zeroed or foreign records take it)
          bool capw = false;
          if (__float_as_uint(e.no_cap) != 0x3F800000u) {  // a scalar compare
            float qmax = qv[0];
#pragma unroll
            for (int i = 1; i < PPT; ++i) qmax = fmaxf(qmax, qv[i]);
            capw = __ballot(qmax >= kBelowCapQ) != 0ull;
          }
          float alv[PPT], wdv[PPT];  // wdv[i] is read only where it was written
#pragma unroll
          for (int i = 0; i < PPT; ++i) alv[i] = __builtin_amdgcn_exp2f(qv[i]);
          if (capw) {
#pragma unroll
            for (int i = 0; i < PPT; ++i) alv[i] = alv[i] < 0.99f ? alv[i] : 0.99f;
          }
          // Pixel 0 runs for every lane, with alpha 0 where it does not blend (1/T and Rg
          // keep their values, the sums get +0): its sums need no clearing per entry.
#pragma unroll
          for (int i = 0; i < PPT; ++i) {
            const bool blends = (!KT || k < kp[i]) && qv[i] > e.thr;
            if (i == 0 || blends) {
              any = any || blends;
              const float al = i == 0 ? (blends ? alv[0] : 0.0f) : alv[i];
              // 1/T_k = (1 - alpha) / T_{k+1}, one rounding; T_k from it by rcp, which
              // does not feed back into the recursion
              const float iTk = fmaf(-al, Tr[i], Tr[i]);
              const float Tk = __builtin_amdgcn_rcpf(iTk);
              const float w = al * Tk;
              gc0 = fmaf(w, g0[i], gc0);
              gc1 = fmaf(w, g1[i], gc1);
              gc2 = fmaf(w, g2[i], gc2);
              // c.g - Rg in one fma chain started from -Rg
              const float dR = fmaf(e.b, g2[i], fmaf(e.g, g1[i], fmaf(e.r, g0[i], -Rg[i])));
              const float dpw = w * dR;  // (alpha T) dR
              wdv[i] = dpw;
              Rg[i] = fmaf(al, dR, Rg[i]);
              Tr[i] = iTk;
              P += dpw;
              const float dpy = dpw * dyv[i];
              Q += dpy;
              V = fmaf(dpy, dyv[i], V);
            }
          }
          if (capw) {
            P = -0.0f;
            Q = -0.0f;
            V = -0.0f;
#pragma unroll
            for (int i = 0; i < PPT; ++i) {
              if ((!KT || k < kp[i]) && qv[i] > e.thr) {
                // the alpha before the cap again (a fresh exp2: not kept live across the body)
                float qi = qv[i];
                asm volatile("" : "+v"(qi));
                const float araw = __builtin_amdgcn_exp2f(qi);
                float dpw = araw < 0.99f ? wdv[i] : 0.0f;
                if (__builtin_expect(araw == 0.99f, 0)) dpw = 0.5f * wdv[i];
                P += dpw;
                const float dpy = dpw * dyv[i];
                Q += dpy;
                V = fmaf(dpy, dyv[i], V);
              }
            }
          }
        } else {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
          const float dy = dyv[i];
          const float q = qv[i];
          if (k < kp[i] && q > e.thr) {
            any = true;
            const float araw = __builtin_amdgcn_exp2f(q);
            const float al = araw < 0.99f ? araw : 0.99f;
            const float om = 1.0f - al;
            const float Tk = Tr[i] * __builtin_amdgcn_rcpf(om);
            const float w = al * Tk;
            gc0 = fmaf(w, g0[i], gc0);
            gc1 = fmaf(w, g1[i], gc1);
            gc2 = fmaf(w, g2[i], gc2);
            const float dR = fmaf(e.b, g2[i], fmaf(e.g, g1[i], fmaf(e.r, g0[i], -Rg[i])));  // c.g - Rg
            // dL/dalpha = T dR; d alpha/d power = araw below the cap, where alpha = araw,
            // so dL/dpower = (alpha T) dR = w dR (one product instead of two)
            const float wd = w * dR;
            Rg[i] = fmaf(al, dR, Rg[i]);  // alpha c.g + (1 - alpha) Rg
            Tr[i] = Tk;
            // min(araw, 0.99): the cotangent passes below the cap, half of it at a tie
            // (where alpha = araw too)
            float dpw = araw < 0.99f ? wd : 0.0f;  // d/d power (natural units)
            if (__builtin_expect(araw == 0.99f, 0)) dpw = 0.5f * wd;
            P += dpw;
            const float dpy = dpw * dy;
            Q += dpy;
            V = fmaf(dpy, dy, V);
          }
        }
        }
        }
        // the column sums; the gradient record's [0] dpw dx, [1] dpw dy, [2] dpw dx^2,
        // [3] dpw dx dy, [4] dpw dy^2, [5] dpw, [6..8] colour follow in the reduce-scatter
        s6[h][0] = P;
        s6[h][1] = Q;
        s6[h][2] = V;
        s6[h][3] = gc0;
        s6[h][4] = gc1;
        s6[h][5] = gc2;
        dxh[h] = dx;
        if (h == 1) pair_level32(s6[0], s6[1], p0);
      }
      // the four-pixel build reduces every group (testing for one with no blending pixel
      // cost more than the reductions it saved: cfg4 217 -> 212 us without the test); the
      // one-pixel build skips groups that blend nothing
      if (!NOCAP && __ballot(any) == 0ull) continue;
      float p1[6];
      pair_level32(s6[2], s6[3], p1);
      const float mine = reduce_scatter_quad9(p0, p1, dxh[0], dxh[1], dxh[2], dxh[3], lane);
      const int vi = quad9_index(lane);
      // the record of entry quad_entry(lane) = 2 bit4 + bit5
      const bool b4 = (lane >> 4) & 1, b5 = (lane >> 5) & 1;
      const int g01 = b5 ? gh[1] : gh[0], g23 = b5 ? gh[3] : gh[2];
      const int gq = b4 ? g23 : g01;
      if (vi < 9 && mine != 0.0f) atomicAdd(grec_at<O32>(grec, gq, vi), mine);
    }
    };
    const uint64_t m = probe_test(pr, rx0, rx1, ry0, ry1);
    if (NOCAP && b0 + 63 < kmin) {
      walk(BoolTag<false>{}, m);
    } else if (NOCAP && b0 < kmin) {
      // the batch straddles the minimum: its entries from kmin up with the test, then (in
      // the same descending order) the ones below without it
      const uint64_t below = (1ull << (kmin - b0)) - 1ull;  // kmin - b0 in 1..63
      walk(BoolTag<true>{}, m & ~below);
      walk(BoolTag<false>{}, m & below);
    } else {
      walk(BoolTag<true>{}, m);
    }
  }
}

// The arrays of a gs_clear_list_t, passed by value.  Workgroup b of nb (64 threads, t the
// thread) zeroes its contiguous
// share of each array's 16-byte-aligned body with non-temporal stores (the lines go to HBM while
// the launch's waves compute, rather than staying dirty in the caches until a later kernel's
// traffic evicts them); workgroup 0 also zeroes the up to three floats before and after it.
struct ClearList {
  float* p[GS_CLEAR_MAX];
  int64_t n[GS_CLEAR_MAX];
};

__device__ inline void clear_list_share(const ClearList& cl, int b, int nb, int t) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
  for (int r = 0; r < GS_CLEAR_MAX; ++r) {
    float* const p = cl.p[r];
    const int64_t n = cl.n[r];
    if (p == nullptr || n <= 0) continue;
    const int64_t lead = (int64_t)((16u - (uint32_t)(reinterpret_cast<uintptr_t>(p) & 15u)) & 15u) / 4;
    const int64_t head = lead < n ? lead : n;
    const int64_t n4 = (n - head) / 4;
    const int64_t per = (n4 + nb - 1) / nb;
    const int64_t c0 = per * b, c1 = c0 + per < n4 ? c0 + per : n4;
    f4v* const v = reinterpret_cast<f4v*>(p + head);
    // four stores per iteration at immediate offsets of one address: the loop's own vector
    // instructions (64-bit address, compare) compete with the launch's arithmetic
    int64_t c = c0 + t;
    for (; c + 192 < c1; c += 256) {
      __builtin_nontemporal_store(z, v + c);
      __builtin_nontemporal_store(z, v + c + 64);
      __builtin_nontemporal_store(z, v + c + 128);
      __builtin_nontemporal_store(z, v + c + 192);
    }
    for (; c < c1; c += 64) __builtin_nontemporal_store(z, v + c);
    if (b == 0) {
      const int64_t tail0 = head + 4 * n4;
      if (t < head) p[t] = 0.0f;
      if (t < n - tail0) p[tail0 + t] = 0.0f;
    }
  }
}

#define GS_BWD_PARAMS                                                                                       \
  const float4 *__restrict__ rec, int num_g, const int32_t *__restrict__ gids, int64_t n_entries,               \
      const int32_t *__restrict__ ranges, int W, int H, int TX, int T, const float *__restrict__ bg,            \
      const ImageCot gc, const float *__restrict__ finalT, const int32_t *__restrict__ ncontrib,               \
      float *__restrict__ grec, const int32_t *__restrict__ order, const gs_window_t *__restrict__ win
#define GS_BWD_ARGS rec, num_g, gids, n_entries, ranges, W, H, TX, T, bg, gc, finalT, ncontrib, grec, order, win

// The backward's two builds.  One pixel per lane (images below 2048 tiles, four waves per
// tile): 64 VGPRs, 8 waves per SIMD, the general body only (the no-cap path's per-entry test
// costs more than it saves with one pixel per lane: cfg0 169 -> 174 us, cfg1 230 -> 236), four
// walked entries per reduce-scatter (skipped when none of them blends a pixel of the wave):
// cfg0 154 -> 142 us, cfg1 210 -> 199 against two.
// Four pixels per lane: the no-cap body, which beats the 64-VGPR build without it at every
// size (cfg2, 8160 tiles: 306 vs 332 us; cfg4, 3600 tiles: 233 vs 248; cfg3: 198 vs 207);
// one body with the cap applied in place and the 1/T state took cfg2 from 310 to 304 us
// (8 % fewer VALU instructions, the copies of the state between two bodies gone).  Its
// reduce-scatter takes four walked entries at a time, which needs 91 VGPRs, so the build
// is scheduled for 5 waves per SIMD (at 6, 80 VGPRs, it spilled): cfg2 285 -> 273 us and
// cfg4 223 -> 214 against two entries at 6 waves per SIMD.  WIN: the default path's chunk
// windows, as the forward read them.
// Each workgroup zeroes its share of the clear list after its walk (stores issued before it
// would hold up its first loads: loads and stores share one wait counter).
template <int PPT, bool WIN, bool O32>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8))) void composite_bwd_kernel(GS_BWD_PARAMS,
                                                                                                     const ClearList cl) {
  composite_bwd_body<PPT, WIN, false, O32>(GS_BWD_ARGS);
  clear_list_share(cl, blockIdx.x, gridDim.x, threadIdx.x);
}
template <bool WIN, bool O32>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(5, 5))) void composite_bwd_wide_kernel(
    GS_BWD_PARAMS, const ClearList cl) {
  composite_bwd_body<4, WIN, true, O32>(GS_BWD_ARGS);
  clear_list_share(cl, blockIdx.x, gridDim.x, threadIdx.x);
}
#undef GS_BWD_PARAMS
#undef GS_BWD_ARGS

// Clears the gradient records (and the 3 background cotangents when given).
__global__ void zero_grads_kernel(float4* __restrict__ p, int64_t n4, float* __restrict__ gbg) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = tid; i < n4; i += stride) p[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (gbg != nullptr && tid < 3) gbg[tid] = 0.0f;
}

// dL/dbackground = sum over pixels of T_final * g (rasterizer.py:244): grid-stride
// partial sums, a block reduction and 3 atomics per block.
__global__ __launch_bounds__(256) void background_grad_kernel(int64_t npix, int W, int H,
                                                              const float* __restrict__ finalT, const ImageCot gc,
                                                              float* __restrict__ gbg) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const float sc = l1_scale(gc, W, H);
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < npix; p += stride) {
    const float t = finalT[p];
    float g0, g1, g2;
    image_cot(gc, sc, p, g0, g1, g2);
    a0 = fmaf(t, g0, a0);
    a1 = fmaf(t, g1, a1);
    a2 = fmaf(t, g2, a2);
  }
  a0 = wave_sum(a0);
  a1 = wave_sum(a1);
  a2 = wave_sum(a2);
  __shared__ float ws[4][3];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) {
    ws[wid][0] = a0;
    ws[wid][1] = a1;
    ws[wid][2] = a2;
  }
  __syncthreads();
  if (threadIdx.x < 3)
    atomicAdd(&gbg[threadIdx.x], (ws[0][threadIdx.x] + ws[1][threadIdx.x]) + (ws[2][threadIdx.x] + ws[3][threadIdx.x]));
}

// Backward schedule.  Every wave of a compositing launch is resident from the start
// (one wave per tile, 8 per SIMD), so a launch lasts as long as its most loaded SIMD;
// tiles differ in walk length by an order of magnitude, and in tile order a SIMD's
// 8 tiles can all be long.  Handing the tiles out longest first (blocks are dispatched
// in index order, round-robin over the XCDs and SIMDs) spreads the long walks over
// all SIMDs, each next to short ones.  The forward pass measures the walk length of
// every tile; the backward walks the same entries (up to the last contributing one),
// so that length is its cost.  tile_order_kernel turns the lengths (written into the
// order array itself) into the permutation, longest first: a counting sort over
// buckets of 8 entries in one workgroup, with the lengths held in LDS.  Beyond
// kOrderMaxTiles tiles the order is the identity.
constexpr int kOrderMaxTiles = 65536;
constexpr int kOrderBuckets = 1024;  // walk lengths <= 4096 -> buckets <= 512

// The same workgroup finishes the fused L1 loss: loss = (sum of the forward's per-workgroup
// partials) / count, the partials added in a fixed order (no atomics: the same value on
// every run).
__global__ __launch_bounds__(1024) void tile_order_kernel(int32_t* __restrict__ order, int T,
                                                          const float* __restrict__ l1_part, int nparts,
                                                          int64_t count, float* __restrict__ l1_loss) {
  __shared__ uint16_t bucket[kOrderMaxTiles];
  __shared__ int start[kOrderBuckets];
  __shared__ int wsum[16];
  __shared__ float fsum[16];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // the workgroup is latency-bound: the first 8 walk lengths and the partials of each round
  // of 8 are requested together, before anything waits for them
  const bool ord = order != nullptr && T <= kOrderMaxTiles;
  uint32_t w0[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int t = tid + 1024 * k;
    w0[k] = ord && t < T ? (uint32_t)order[t] : 0u;
  }
  if (l1_part != nullptr) {
    float a = 0.0f;
    for (int i0 = 0; i0 < nparts; i0 += 8 * 1024) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = i0 + tid + 1024 * k;
        v[k] = i < nparts ? l1_part[i] : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) a += v[k];
    }
    a = wave_sum(a);
    if (lane == 0) fsum[wid] = a;
    __syncthreads();
    if (tid == 0) {
      float t = 0.0f;
      for (int w = 0; w < 16; ++w) t += fsum[w];
      l1_loss[0] = t / (float)count;  // jnp.mean: the sum over the count
    }
  }
  if (order == nullptr) return;
  if (T > kOrderMaxTiles) {
    for (int t = tid; t < T; t += 1024) order[t] = t;
    return;
  }
  start[tid] = 0;
  __syncthreads();
  auto count_tile = [&](int t, uint32_t w) {
    const int c = (int)max(w & 0xFFFFu, w >> 16);  // the longer of the tile's (one or two) walks
    const int bk = min(c >> 3, kOrderBuckets - 1);
    bucket[t] = (uint16_t)bk;
    atomicAdd(&start[bk], 1);
  };
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (tid + 1024 * k < T) count_tile(tid + 1024 * k, w0[k]);
  for (int t = tid + 8 * 1024; t < T; t += 1024) count_tile(t, (uint32_t)order[t]);
  __syncthreads();
  // exclusive scan over buckets in descending order: thread j owns bucket 1023 - j
  const int own = start[kOrderBuckets - 1 - tid];
  int x = own;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wid] = x;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wid; ++w) before += wsum[w];
  start[kOrderBuckets - 1 - tid] = before + x - own;
  __syncthreads();
  for (int t = tid; t < T; t += 1024) order[atomicAdd(&start[bucket[t]], 1)] = t;
}

// Record byte offsets (gid * 48) fit the 32-bit offset register of scalar loads.
inline bool rec_offsets_fit(int64_t n) { return n * (int64_t)(kRec * 4) <= (int64_t)0xFFFFFFFF - 64; }

// Large images have enough tiles to fill the GPU with one wave per tile.
inline int pick_ppt(int T) { return T >= 2048 ? 4 : 1; }
// Tiles from which the forward gives a tile one wave (four pixels per lane); below that (and
// from 2048 tiles) two waves of eight rows each: at 3600 tiles a launch holds 3-4 waves per
// SIMD, and halving the work units evens them out (cfg4 forward 189 -> 176 us) where at
// 8160 tiles the duplicated per-entry work costs more than it balances (227 -> 255 us).
constexpr int kFwdOneWaveTiles = 6 * 1024;

}  // namespace
}  // namespace gs

using namespace gs;

namespace gs {
namespace {
// thr = L - 512 and the last 512 ids of an L-slot list (no clamp for L < 512)
__global__ __launch_bounds__(512) void window_list_kernel(const int32_t* __restrict__ gids, int64_t L,
                                                          gs_window_t* __restrict__ win) {
  const int i = threadIdx.x;
  if (i == 0) win->thr = L >= kBlock ? L - kBlock : INT64_MAX;
  if (i < 2) win->reserved[i] = 0;
  win->ids[i] = L >= kBlock ? gids[L - kBlock + i] : 0;
}
}  // namespace
}  // namespace gs

extern "C" int gs_window_from_list(void* stream, const int32_t* sorted_gids, int64_t n_entries,
                                   gs_window_t* window) {
  GS_REQUIRE(n_entries >= 0 && window != nullptr, "gs_window_from_list: bad arguments");
  GS_REQUIRE(n_entries < kBlock || sorted_gids != nullptr, "gs_window_from_list: NULL sorted_gids");
  hipLaunchKernelGGL(window_list_kernel, dim3(1), dim3(kBlock), 0, (hipStream_t)stream, sorted_gids, n_entries,
                     window);
  GS_LAUNCH_CHECK("window_list_kernel");
  return GS_OK;
}

namespace {
// Floats of the l1_out array of the fused L1 loss: the loss, then one partial sum per
// compositing workgroup (at most four per tile cell of the launch grid).
int64_t l1_out_floats(int width, int height) {
  const int TX = (width + kTile - 1) / kTile, TY = (height + kTile - 1) / kTile;
  return 1 + 4 * (int64_t)tile_blocks(TX, TY);
}

int composite_fwd_run(const char* name, void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                      int64_t n_entries, const int32_t* ranges, int width, int height, const float* background,
                      float* image, float* final_T, int32_t* n_contrib, int32_t* tile_order, float* clear_records,
                      const gs_window_t* window, const SBLists* sbl, int32_t* gids_out,
                      const float* l1_target = nullptr, float* l1_out = nullptr) {
  GS_REQUIRE(n >= 0 && n < ((int64_t)1 << 31), "%s: n out of range", name);
  GS_REQUIRE(n_entries >= 0, "%s: n_entries must be >= 0", name);
  GS_REQUIRE(width > 0 && height > 0, "%s: bad image size %dx%d", name, width, height);
  GS_REQUIRE(ranges && background && image, "%s: NULL argument", name);
  GS_REQUIRE(n == 0 || n_entries == 0 || (records && sorted_gids), "%s: NULL records/gids", name);
  const int TX = (width + kTile - 1) / kTile, TY = (height + kTile - 1) / kTile;
  const int T = TX * TY;
  const int nblk = tile_blocks(TX, TY);
  hipStream_t s = (hipStream_t)stream;
  GS_REQUIRE(clear_records == nullptr || ((uintptr_t)clear_records & 15) == 0,
             "%s: clear_records must be 16-byte aligned", name);
  const int64_t n4_clear = clear_records ? n * kRec / 4 : 0;  // kRec = 12: whole float4s
  GS_REQUIRE((l1_target == nullptr) == (l1_out == nullptr), "%s: l1_target and l1_out go together", name);
  float* l1_part = l1_out ? l1_out + 1 : nullptr;
  const SBLists none{};
#define GS_FWD_LAUNCH2(PPT, WPT, WIN, O32, SB)                                                                  \
  hipLaunchKernelGGL((composite_fwd_kernel<PPT, WIN, O32, SB>), dim3(nblk * (WPT)), dim3(64), 0, s,             \
                     (const float4*)records, (int)n, sorted_gids, n_entries, ranges, width, height, TX, T,        \
                     background, image, final_T, n_contrib, tile_order, (float4*)clear_records, n4_clear, window, \
                     SB ? *sbl : none, gids_out, l1_target, l1_part)
#define GS_FWD_LAUNCH1(PPT, WPT, WIN, O32) \
  if (sbl) GS_FWD_LAUNCH2(PPT, WPT, WIN, O32, true); else GS_FWD_LAUNCH2(PPT, WPT, WIN, O32, false)
#define GS_FWD_LAUNCH(PPT, WPT, WIN) \
  if (o32) { GS_FWD_LAUNCH1(PPT, WPT, WIN, true); } else { GS_FWD_LAUNCH1(PPT, WPT, WIN, false); }
  const bool win = window != nullptr, o32 = rec_offsets_fit(n);
  if (pick_ppt(T) == 4 && T >= kFwdOneWaveTiles) {
    if (win) { GS_FWD_LAUNCH(4, 1, true); } else { GS_FWD_LAUNCH(4, 1, false); }
  } else if (pick_ppt(T) == 4) {
    if (win) { GS_FWD_LAUNCH(2, 2, true); } else { GS_FWD_LAUNCH(2, 2, false); }
  } else {
    if (win) { GS_FWD_LAUNCH(1, 4, true); } else { GS_FWD_LAUNCH(1, 4, false); }
  }
#undef GS_FWD_LAUNCH
#undef GS_FWD_LAUNCH1
#undef GS_FWD_LAUNCH2
  GS_LAUNCH_CHECK("composite_fwd_kernel");
  if (tile_order || l1_out) {
    const int wpt = pick_ppt(T) == 4 ? (T >= kFwdOneWaveTiles ? 1 : 2) : 4;
    hipLaunchKernelGGL(tile_order_kernel, dim3(1), dim3(1024), 0, s, tile_order, T, l1_part, nblk * wpt,
                       (int64_t)width * height * 3, l1_out);
    GS_LAUNCH_CHECK("tile_order_kernel");
  }
  return GS_OK;
}
}  // namespace

extern "C" int gs_composite_fwd(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                                int64_t n_entries, const int32_t* ranges, int width, int height,
                                const float* background, float* image, float* final_T, int32_t* n_contrib,
                                int32_t* tile_order, float* clear_records, const gs_window_t* window) {
  return composite_fwd_run("gs_composite_fwd", stream, n, records, sorted_gids, n_entries, ranges, width, height,
                           background, image, final_T, n_contrib, tile_order, clear_records, window, nullptr,
                           nullptr);
}

extern "C" int gs_composite_fwd_deferred(void* stream, int64_t n, const float* records, int32_t* sorted_gids,
                                         int64_t capacity, const int32_t* ranges, const int32_t* stats,
                                         const void* bin_workspace, size_t bin_workspace_bytes, int width, int height,
                                         const float* background, float* image, float* final_T, int32_t* n_contrib,
                                         int32_t* tile_order, float* clear_records, const gs_window_t* window) {
  GS_REQUIRE(capacity > 0, "gs_composite_fwd_deferred: capacity must be > 0 (got %lld)", (long long)capacity);
  GS_REQUIRE(stats != nullptr && (n == 0 || sorted_gids != nullptr), "gs_composite_fwd_deferred: NULL argument");
  SBLists sbl;
  const int rc = superblock_lists(n, width, height, capacity, bin_workspace, bin_workspace_bytes, stats, &sbl);
  if (rc != GS_OK) return rc;
  return composite_fwd_run("gs_composite_fwd_deferred", stream, n, records, sorted_gids, capacity, ranges, width,
                           height, background, image, final_T, n_contrib, tile_order, clear_records, window, &sbl,
                           sorted_gids);
}

extern "C" int64_t gs_composite_l1_out_size(int width, int height) {
  return width > 0 && height > 0 ? l1_out_floats(width, height) : 0;
}

extern "C" int gs_composite_fwd_deferred_l1(void* stream, int64_t n, const float* records, int32_t* sorted_gids,
                                            int64_t capacity, const int32_t* ranges, const int32_t* stats,
                                            const void* bin_workspace, size_t bin_workspace_bytes, int width,
                                            int height, const float* background, float* image, float* final_T,
                                            int32_t* n_contrib, int32_t* tile_order, float* clear_records,
                                            const gs_window_t* window, const float* l1_target, float* l1_out) {
  GS_REQUIRE(capacity > 0, "gs_composite_fwd_deferred_l1: capacity must be > 0 (got %lld)", (long long)capacity);
  GS_REQUIRE(stats != nullptr && (n == 0 || sorted_gids != nullptr), "gs_composite_fwd_deferred_l1: NULL argument");
  GS_REQUIRE(l1_target != nullptr && l1_out != nullptr, "gs_composite_fwd_deferred_l1: NULL l1_target or l1_out");
  SBLists sbl;
  const int rc = superblock_lists(n, width, height, capacity, bin_workspace, bin_workspace_bytes, stats, &sbl);
  if (rc != GS_OK) return rc;
  return composite_fwd_run("gs_composite_fwd_deferred_l1", stream, n, records, sorted_gids, capacity, ranges, width,
                           height, background, image, final_T, n_contrib, tile_order, clear_records, window, &sbl,
                           sorted_gids, l1_target, l1_out);
}

namespace {
int composite_bwd_run(const char* name, void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                      int64_t n_entries, const int32_t* ranges, int width, int height, const float* background,
                      const ImageCot& gc, const float* final_T, const int32_t* n_contrib,
                      const int32_t* tile_order, float* grad_records, float* grad_background, int accumulate,
                      const gs_window_t* window, const gs_clear_list_t* clear) {
  GS_REQUIRE(n >= 0 && n < ((int64_t)1 << 31), "%s: n out of range", name);
  ClearList cl{};
  if (clear != nullptr) {
    for (int r = 0; r < GS_CLEAR_MAX; ++r) {
      GS_REQUIRE(clear->count[r] >= 0, "%s: clear list entry %d has a negative count", name, r);
      GS_REQUIRE(clear->count[r] == 0 || clear->ptr[r] != nullptr, "%s: clear list entry %d is NULL", name, r);
      cl.p[r] = clear->count[r] > 0 ? clear->ptr[r] : nullptr;
      cl.n[r] = clear->count[r];
    }
  }
  GS_REQUIRE(n_entries >= 0, "%s: n_entries must be >= 0", name);
  GS_REQUIRE(width > 0 && height > 0, "%s: bad image size %dx%d", name, width, height);
  GS_REQUIRE(ranges && background && final_T && n_contrib, "%s: NULL argument", name);
  GS_REQUIRE(gc.tgt != nullptr ? (gc.img != nullptr && gc.cot != nullptr) : gc.gimg != nullptr,
             "%s: NULL image cotangent", name);
  GS_REQUIRE(n == 0 || n_entries == 0 || (records && sorted_gids && grad_records), "%s: NULL records/gids", name);
  hipStream_t s = (hipStream_t)stream;
  if ((n > 0 && !accumulate) || grad_background) {
    // clears the records unless accumulating, and the background cotangent
    hipLaunchKernelGGL(zero_grads_kernel, dim3(accumulate ? 1 : 1024), dim3(256), 0, s, (float4*)grad_records,
                       accumulate ? (int64_t)0 : n * kRec / 4, grad_background);
    GS_LAUNCH_CHECK("zero_grads_kernel");
  }
  if (grad_background) {
    const int64_t npix = (int64_t)width * height;
    hipLaunchKernelGGL(background_grad_kernel, dim3(std::min<int64_t>(1024, div_up(npix, 256))), dim3(256), 0, s,
                       npix, width, height, final_T, gc, grad_background);
    GS_LAUNCH_CHECK("background_grad_kernel");
  }
  const int TX = (width + kTile - 1) / kTile, TY = (height + kTile - 1) / kTile;
  const int T = TX * TY;
  const int nblk = tile_blocks(TX, TY);
#define GS_BWD_LAUNCH(KERNEL, WPT)                                                                                  \
  hipLaunchKernelGGL(KERNEL, dim3(nblk * (WPT)), dim3(64), 0, s, (const float4*)records, (int)n, sorted_gids, n_entries, \
                     ranges, width, height, TX, T, background, gc, final_T, n_contrib, grad_records,                   \
                     tile_order, window, cl)
  const bool win = window != nullptr, o32 = rec_offsets_fit(n);
  if (pick_ppt(T) == 4) {
    if (o32) {
      if (win) GS_BWD_LAUNCH((composite_bwd_wide_kernel<true, true>), 1);
      else GS_BWD_LAUNCH((composite_bwd_wide_kernel<false, true>), 1);
    } else {
      if (win) GS_BWD_LAUNCH((composite_bwd_wide_kernel<true, false>), 1);
      else GS_BWD_LAUNCH((composite_bwd_wide_kernel<false, false>), 1);
    }
  } else {
    if (o32) {
      if (win) GS_BWD_LAUNCH((composite_bwd_kernel<1, true, true>), 4);
      else GS_BWD_LAUNCH((composite_bwd_kernel<1, false, true>), 4);
    } else {
      if (win) GS_BWD_LAUNCH((composite_bwd_kernel<1, true, false>), 4);
      else GS_BWD_LAUNCH((composite_bwd_kernel<1, false, false>), 4);
    }
  }
#undef GS_BWD_LAUNCH
  GS_LAUNCH_CHECK("composite_bwd_kernel");
  return GS_OK;
}
}  // namespace

extern "C" int gs_composite_bwd(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                                int64_t n_entries, const int32_t* ranges, int width, int height,
                                const float* background, const float* grad_image, const float* final_T,
                                const int32_t* n_contrib, const int32_t* tile_order, float* grad_records,
                                float* grad_background, int accumulate, const gs_window_t* window,
                                const gs_clear_list_t* clear) {
  const ImageCot gc{grad_image, nullptr, nullptr, nullptr};
  return composite_bwd_run("gs_composite_bwd", stream, n, records, sorted_gids, n_entries, ranges, width, height,
                           background, gc, final_T, n_contrib, tile_order, grad_records, grad_background, accumulate,
                           window, clear);
}

extern "C" int gs_composite_bwd_l1(void* stream, int64_t n, const float* records, const int32_t* sorted_gids,
                                   int64_t n_entries, const int32_t* ranges, int width, int height,
                                   const float* background, const float* grad_image, const float* image,
                                   const float* l1_target, const float* l1_cot, const float* final_T,
                                   const int32_t* n_contrib, const int32_t* tile_order, float* grad_records,
                                   float* grad_background, int accumulate, const gs_window_t* window,
                                   const gs_clear_list_t* clear) {
  GS_REQUIRE(image != nullptr && l1_target != nullptr && l1_cot != nullptr,
             "gs_composite_bwd_l1: NULL image, l1_target or l1_cot");
  const ImageCot gc{grad_image, image, l1_target, l1_cot};
  return composite_bwd_run("gs_composite_bwd_l1", stream, n, records, sorted_gids, n_entries, ranges, width,
                           height, background, gc, final_T, n_contrib, tile_order, grad_records, grad_background,
                           accumulate, window, clear);
}
