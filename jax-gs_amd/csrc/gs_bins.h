// Superblock lists of the tile binning, shared by the binning (gs_binning.hip) and the
// compositing forward (gs_composite.hip).
//
// A superblock is 8x8 tiles.  The binning lists, per superblock, the packed words of the
// Gaussians whose tile rectangle meets it, in (depth bucket, id) order; a tile's entries
// are exactly the words of its superblock's list whose rectangle holds the tile, in the
// list's order (rasterizer.py:12-116 sorts them by (tile, bucket, id)).  The deferred
// binning (gs_bin_deferred) stops there and leaves the entry list to the compositing
// forward, which walks the superblock list of each tile itself and writes the entries it
// meets -- the prefix the backward replays -- unless the entry list has to exist in full
// (the default path's clamped chunk window reads it, or the entries exceed the capacity).
#pragma once

#include "gs_common.h"

namespace gs {

constexpr int kSB = 8;  // superblock = 8x8 tiles

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

// A deferred binning's superblock lists, as the compositing forward reads them.  A
// superblock's list is cut into chunks of 256 words (4 steps of 64); its chunks are
// chunk_base[s] .. chunk_base[s+1]-1, chunk c starting at word ranges[s] + 256 (c -
// chunk_base[s]).  masks[(c * 64 + u) * 4 + k] says which words of step k of chunk c hold
// tile u of the superblock (u = 8 row + column within it; bit l: word 64 k + l): the
// binning's count sweep computes them anyway, and the forward reads them in place of the
// words.
struct SBLists {
  const uint64_t* words;        // packed words, grouped by superblock
  const int32_t* ranges;        // [S+1]: superblock s's words are words[ranges[s] .. ranges[s+1])
  const uint32_t* chunk_base;   // [S+1]: first chunk of each superblock
  const uint64_t* masks;        // [n_chunks][64][4] step masks
  int64_t n_chunks;             // chunks the masks have room for
  int64_t n_words;              // length of words
  int SX;                       // superblocks per row
  const int32_t* stats;         // the binning's stats
};

// Images of fewer tiles are composited with four waves per tile (one pixel per lane), each
// of which would queue the tile's entries from the superblock lists itself; with small
// Gaussians a superblock list holds 15-50 words per entry of a tile, and the forward then
// costs more than the write sweep saves (cfg1: 124 -> 194 us against 93 -> 80 us).
constexpr int kDeferMinTiles = 2048;

// Whether a deferred binning leaves the entry list unwritten: the image has at least
// kDeferMinTiles tiles, every entry fits the capacity and no chunk of the default path reads
// the clamped window.  The tile scan decides and records it in the stats
// (GS_STAT_ENTRIES_DEFERRED, 0 from every other binning); the write sweep and the compositing
// forward read the flag.
__host__ __device__ inline bool defer_entries(int T, int64_t entries, int64_t cap, bool clamped) {
  return T >= kDeferMinTiles && entries >= 0 && entries <= cap && !clamped;
}
__device__ inline bool entries_deferred(const int32_t* __restrict__ stats) {
  return stats[GS_STAT_ENTRIES_DEFERRED] != 0;
}

// The superblock lists inside a gs_bin_deferred workspace (the same n, image size and
// capacity as that call).  Returns GS_OK, or GS_ERR_INVALID for a workspace smaller than
// the binning's.
int superblock_lists(int64_t n, int width, int height, int64_t capacity, const void* workspace,
                     size_t workspace_bytes, const int32_t* stats, SBLists* out);

}  // namespace gs
