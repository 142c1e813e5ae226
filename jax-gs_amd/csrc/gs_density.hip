// Densify-and-prune over the static-capacity Gaussian arrays on gfx950.
//
// Reference: jax_gs/training/density.py:98-211 (densify_and_prune) and :63-67
// (_reset_accumulators).  With M the capacity:
//   prune   = active & (sigmoid(opacity) < min_opacity | max exp(scale) > 0.1 extent
//                       | max_radii > max_screen_size);  after = active & !prune
//   avg     = denom > 0 ? grad_accum / denom : 0
//   densify = avg >= grad_threshold & after;  split = densify & max exp(scale) > 0.01 extent;
//   clone   = densify & !split;  both cleared unless densify_enabled and
//             #clone + #split <= #(!after)
//   the k-th empty slot (!after, in index order) takes a copy of the k-th clone source
//   (index order), then of the (k - #clone)-th split source; copies and split sources get
//   scale -= log(1.6) and mean += noise * exp(new scale) when split; active = after |
//   filled slots; grad_accum and denom are cleared (max_radii is kept, as the reference).
// Every array whose leading dimension is the capacity is moved the same way (the
// optimizer moments).  The reference gathers every array through an index map that is
// the identity except at the filled slots; here only the filled slots are written: their
// sources are active after pruning, so no source is also a destination and the copy is
// safe in place.
//
// Kernels: flags (per Gaussian: after / clone / split / pruned, workgroup counts), one
// workgroup scan of the counts (offsets, totals, the capacity check), routing (ranks by
// ballot + mbcnt: sources and the filled slots scattered by rank, mask and accumulators
// written), the moves (one thread per value of a filled slot's rows) and the split
// (one thread per split and component: the copy and its source).
#include "gs_common.h"

#include <cmath>

namespace gs {
namespace {

constexpr int kDenBlock = 1024;  // Gaussians per workgroup of the flag and route passes
constexpr int kDenMaxArrays = 15;  // 5 parameter arrays + up to 10 moment arrays

enum { kAfter = 1, kClone = 2, kSplit = 4, kPruned = 8 };

struct DenArrays {
  float* a[kDenMaxArrays];
  int row[kDenMaxArrays];  // floats per Gaussian
  int off[kDenMaxArrays];  // first value of the array in a slot's concatenated rows
  int n, per_slot;         // arrays, values per slot
};

struct DenParams {
  float grad_threshold, min_opacity, max_scale_prune, min_scale_split, max_screen, log16;
  int densify_enabled;
};

// control words written by the scan (the caller's counts[5] when given): [0] clones
// [1] splits [2] pruned [3] available (empty slots after pruning) [4] densified (0/1)
__global__ __launch_bounds__(kDenBlock) void density_flags_kernel(
    int64_t M, const float* __restrict__ scales, const float* __restrict__ opacities,
    const uint8_t* __restrict__ active, const float* __restrict__ grad_accum, const int32_t* __restrict__ denom,
    const float* __restrict__ max_radii, DenParams P, uint8_t* __restrict__ flags, int32_t* __restrict__ bcount) {
  const int64_t i = (int64_t)blockIdx.x * kDenBlock + threadIdx.x;
  uint8_t f = 0;
  if (i < M) {
    const bool act = active[i] != 0;
    const float sig = det_sigmoidf(opacities[i]);
    const float ms = fmaxf(fmaxf(det_expf(scales[3 * i]), det_expf(scales[3 * i + 1])), det_expf(scales[3 * i + 2]));
    const bool prune = act && (sig < P.min_opacity || ms > P.max_scale_prune || max_radii[i] > P.max_screen);
    const bool after = act && !prune;
    const int32_t d = denom[i];
    const float avg = d > 0 ? grad_accum[i] / (float)d : 0.0f;
    const bool dens = after && avg >= P.grad_threshold;
    const bool split = dens && ms > P.min_scale_split;
    f = (after ? kAfter : 0) | (dens && !split ? kClone : 0) | (split ? kSplit : 0) | (prune ? kPruned : 0);
    flags[i] = f;
  }
  // workgroup counts of empty slots, clone and split candidates, pruned
  __shared__ int cnt[4][kDenBlock / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool valid = i < M;
  const int c0 = __popcll(__ballot(valid && !(f & kAfter)));
  const int c1 = __popcll(__ballot((f & kClone) != 0));
  const int c2 = __popcll(__ballot((f & kSplit) != 0));
  const int c3 = __popcll(__ballot((f & kPruned) != 0));
  if (lane == 0) {
    cnt[0][w] = c0;
    cnt[1][w] = c1;
    cnt[2][w] = c2;
    cnt[3][w] = c3;
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    int s = 0;
    for (int k = 0; k < kDenBlock / 64; ++k) s += cnt[threadIdx.x][k];
    bcount[(int64_t)blockIdx.x * 4 + threadIdx.x] = s;
  }
}

// One workgroup: exclusive scan of the per-workgroup counts (in place) and the totals.
__global__ __launch_bounds__(1024) void density_scan_kernel(int nb, int32_t* __restrict__ bcount,
                                                            int densify_enabled, int32_t* __restrict__ ctl) {
  __shared__ int32_t carry[4];
  __shared__ int32_t wsum[4][16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid < 4) carry[tid] = 0;
  __syncthreads();
  for (int base = 0; base < nb; base += 1024) {
    const int b = base + tid;
    int v[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = b < nb ? bcount[(int64_t)b * 4 + c] : 0;
    int x[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      x[c] = v[c];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x[c], o, 64);
        if (lane >= o) x[c] += y;
      }
      if (lane == 63) wsum[c][w] = x[c];
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      int before = carry[c];
      for (int k = 0; k < w; ++k) before += wsum[c][k];
      if (b < nb) bcount[(int64_t)b * 4 + c] = before + x[c] - v[c];
    }
    __syncthreads();
    if (tid < 4) {
      int s = 0;
      for (int k = 0; k < 16; ++k) s += wsum[tid][k];
      carry[tid] += s;
    }
    __syncthreads();
  }
  if (tid == 0) {
    const int avail = carry[0], nc = carry[1], ns = carry[2];
    const int can = densify_enabled && (int64_t)nc + ns <= avail;
    ctl[0] = can ? nc : 0;
    ctl[1] = can ? ns : 0;
    ctl[2] = carry[3];
    ctl[3] = avail;
    ctl[4] = can;
  }
}

// Rank of this thread's flag among the set flags of the Gaussians before it.
__device__ inline int block_rank(bool set, int* wbase, int which, int lane, int w) {
  const uint64_t m = __ballot(set);
  const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
  int before = 0;
  for (int k = 0; k < w; ++k) before += wbase[which * (kDenBlock / 64) + k];
  return before + below;
}

__global__ __launch_bounds__(kDenBlock) void density_route_kernel(
    int64_t M, const uint8_t* __restrict__ flags, const int32_t* __restrict__ boff, const int32_t* __restrict__ ctl,
    int32_t* __restrict__ clone_src, int32_t* __restrict__ split_src, int32_t* __restrict__ dest_slot,
    uint8_t* __restrict__ active, float* __restrict__ grad_accum, int32_t* __restrict__ denom) {
  __shared__ int wcnt[3 * (kDenBlock / 64)];
  const int64_t i = (int64_t)blockIdx.x * kDenBlock + threadIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint8_t f = i < M ? flags[i] : (uint8_t)kAfter;
  const int can = ctl[4];
  const bool is_empty = !(f & kAfter), is_clone = can && (f & kClone), is_split = can && (f & kSplit);
  const uint64_t be = __ballot(is_empty), bc = __ballot(is_clone), bs = __ballot(is_split);
  if (lane == 0) {
    wcnt[0 * (kDenBlock / 64) + w] = __popcll(be);
    wcnt[1 * (kDenBlock / 64) + w] = __popcll(bc);
    wcnt[2 * (kDenBlock / 64) + w] = __popcll(bs);
  }
  __syncthreads();
  const int re = (int)boff[(int64_t)blockIdx.x * 4 + 0] + block_rank(is_empty, wcnt, 0, lane, w);
  const int rc = (int)boff[(int64_t)blockIdx.x * 4 + 1] + block_rank(is_clone, wcnt, 1, lane, w);
  const int rs = (int)boff[(int64_t)blockIdx.x * 4 + 2] + block_rank(is_split, wcnt, 2, lane, w);
  if (i >= M) return;
  if (is_clone) clone_src[rc] = (int32_t)i;
  if (is_split) split_src[rs] = (int32_t)i;
  if (is_empty && re < ctl[0] + ctl[1]) dest_slot[re] = (int32_t)i;
  active[i] = (f & kAfter) ? 1 : 0;
  grad_accum[i] = 0.0f;
  denom[i] = 0;
}

// Filled slot of rank r (the r-th empty slot) takes a copy of its source.  Work item
// (r, j) copies value j of the slot's concatenated rows (every array, row after row),
// so consecutive threads copy consecutive values of one row; the grid strides over
// (filled slots) x (values per slot).
__global__ __launch_bounds__(256) void density_move_kernel(DenArrays A, const int32_t* __restrict__ dest_slot,
                                                           const int32_t* __restrict__ clone_src,
                                                           const int32_t* __restrict__ split_src,
                                                           const int32_t* __restrict__ ctl,
                                                           uint8_t* __restrict__ active) {
  const int nc = ctl[0];
  const int64_t items = (int64_t)(ctl[0] + ctl[1]) * A.per_slot;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < items; it += stride) {
    // 32-bit division when the item index fits (always below 2^31 / 177 slots of SH3)
    const int r = it < 0x7fffffff ? (int)((uint32_t)it / (uint32_t)A.per_slot) : (int)(it / A.per_slot);
    const int j = (int)(it - (int64_t)r * A.per_slot);
    int k = 0;
#pragma unroll
    for (int q = 1; q < kDenMaxArrays; ++q)
      if (q < A.n && j >= A.off[q]) k = q;
    const int L = A.row[k], o = j - A.off[k];
    const int64_t i = dest_slot[r];
    const int64_t src = r >= nc ? split_src[r - nc] : clone_src[r];
    float* __restrict__ a = A.a[k];
    a[i * L + o] = a[src * L + o];
    if (j == 0) active[i] = 1;
  }
}

// The split (after the copies): copy and source get scale - log(1.6) and
// mean + noise * exp(new scale); one thread per (split, component).
__global__ __launch_bounds__(256) void density_split_kernel(float* __restrict__ means, float* __restrict__ scales,
                                                            const int32_t* __restrict__ dest_slot,
                                                            const int32_t* __restrict__ split_src,
                                                            const int32_t* __restrict__ ctl,
                                                            const float* __restrict__ noise, float log16) {
  const int nc = ctl[0];
  const int64_t items = (int64_t)ctl[1] * 3;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < items; it += stride) {
    const int q = (int)(it / 3), c = (int)(it - (int64_t)q * 3);
    const int64_t i = dest_slot[nc + q], src = split_src[q];
    const float sn = scales[3 * src + c] - log16;  // the copy's scale equals the source's
    scales[3 * i + c] = sn;
    scales[3 * src + c] = sn;
    means[3 * i + c] = means[3 * i + c] + noise[3 * i + c] * det_expf(sn);
    means[3 * src + c] = means[3 * src + c] + noise[3 * src + c] * det_expf(sn);
  }
}

// density.py:69-93: opacity logits of active Gaussians set to logit(reset_val).
__global__ __launch_bounds__(256) void reset_opacity_kernel(int64_t M, const uint8_t* __restrict__ active,
                                                            float value, float* __restrict__ opacities) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < M && active[i]) opacities[i] = value;
}

struct DenLayout {
  int64_t nb;
  size_t flags, bcount, ctl, clone_src, split_src, dest_slot, total;
};

DenLayout den_layout(int64_t M) {
  DenLayout L;
  L.nb = div_up(M, kDenBlock);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) & ~(size_t)255;
    return at;
  };
  L.flags = take((size_t)M);
  L.bcount = take((size_t)L.nb * 4 * sizeof(int32_t));
  L.ctl = take(8 * sizeof(int32_t));
  L.clone_src = take((size_t)M * sizeof(int32_t));
  L.split_src = take((size_t)M * sizeof(int32_t));
  L.dest_slot = take((size_t)M * sizeof(int32_t));
  L.total = off;
  return L;
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" size_t gs_densify_workspace_size(int64_t capacity) {
  return capacity > 0 ? den_layout(capacity).total : 0;
}

extern "C" int gs_densify_and_prune(void* stream, int64_t capacity, int sh_k, float* means, float* scales,
                                    float* quats, float* opacities, float* sh_coeffs, int num_moments,
                                    float* const* moments, uint8_t* active, float* grad_accum, int32_t* denom,
                                    const float* max_radii, const float* noise, int densify_enabled,
                                    double grad_threshold, double min_opacity, double extent,
                                    double max_screen_size, void* workspace, size_t workspace_bytes,
                                    int32_t* counts) {
  GS_REQUIRE(capacity > 0 && capacity < ((int64_t)1 << 31), "gs_densify_and_prune: capacity out of range");
  GS_REQUIRE(sh_k >= 1, "gs_densify_and_prune: bad sh_k %d", sh_k);
  GS_REQUIRE(means && scales && quats && opacities && sh_coeffs && active && grad_accum && denom && max_radii &&
                 noise && workspace,
             "gs_densify_and_prune: NULL argument");
  GS_REQUIRE(num_moments % 5 == 0 && num_moments >= 0 && num_moments <= 10,
             "gs_densify_and_prune: num_moments must be 0, 5 or 10");
  GS_REQUIRE(num_moments == 0 || moments, "gs_densify_and_prune: NULL moments");
  const DenLayout L = den_layout(capacity);
  GS_REQUIRE(workspace_bytes >= L.total, "gs_densify_and_prune: workspace of %zu bytes, %zu needed",
             workspace_bytes, L.total);
  DenArrays A{};
  float* params[5] = {means, scales, quats, opacities, sh_coeffs};
  const int rows[5] = {3, 3, 4, 1, 3 * sh_k};
  for (int k = 0; k < 5; ++k) {
    A.a[k] = params[k];
    A.row[k] = rows[k];
  }
  for (int j = 0; j < num_moments; ++j) {
    GS_REQUIRE(moments[j] != nullptr, "gs_densify_and_prune: NULL moment array %d", j);
    A.a[5 + j] = moments[j];
    A.row[5 + j] = rows[j % 5];
  }
  A.n = 5 + num_moments;
  A.per_slot = 0;
  for (int k = 0; k < A.n; ++k) {
    A.off[k] = A.per_slot;
    A.per_slot += A.row[k];
  }
  DenParams P;
  // Python floats of the reference, rounded once to float32 where they meet float32 data
  P.grad_threshold = (float)grad_threshold;
  P.min_opacity = (float)min_opacity;
  P.max_scale_prune = (float)(0.1 * extent);
  P.min_scale_split = (float)(0.01 * extent);
  P.max_screen = (float)max_screen_size;
  P.log16 = (float)std::log(1.6);
  P.densify_enabled = densify_enabled != 0;
  char* ws = (char*)workspace;
  uint8_t* flags = (uint8_t*)(ws + L.flags);
  int32_t* bcount = (int32_t*)(ws + L.bcount);
  int32_t* ctl = counts ? counts : (int32_t*)(ws + L.ctl);
  int32_t* clone_src = (int32_t*)(ws + L.clone_src);
  int32_t* split_src = (int32_t*)(ws + L.split_src);
  int32_t* dest_slot = (int32_t*)(ws + L.dest_slot);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)L.nb);
  hipLaunchKernelGGL(density_flags_kernel, grid, dim3(kDenBlock), 0, s, capacity, scales, opacities, active,
                     grad_accum, denom, max_radii, P, flags, bcount);
  GS_LAUNCH_CHECK("density_flags_kernel");
  hipLaunchKernelGGL(density_scan_kernel, dim3(1), dim3(1024), 0, s, (int)L.nb, bcount, P.densify_enabled, ctl);
  GS_LAUNCH_CHECK("density_scan_kernel");
  hipLaunchKernelGGL(density_route_kernel, grid, dim3(kDenBlock), 0, s, capacity, flags, bcount, ctl, clone_src,
                     split_src, dest_slot, active, grad_accum, denom);
  GS_LAUNCH_CHECK("density_route_kernel");
  // the number of filled slots is known on the device only: fixed grids that stride
  hipLaunchKernelGGL(density_move_kernel, dim3(8192), dim3(256), 0, s, A, dest_slot, clone_src, split_src, ctl,
                     active);
  GS_LAUNCH_CHECK("density_move_kernel");
  hipLaunchKernelGGL(density_split_kernel, dim3(1024), dim3(256), 0, s, means, scales, dest_slot, split_src, ctl,
                     noise, P.log16);
  GS_LAUNCH_CHECK("density_split_kernel");
  return GS_OK;
}

extern "C" int gs_reset_opacities(void* stream, int64_t capacity, const uint8_t* active, double reset_value,
                                  float* opacities) {
  GS_REQUIRE(capacity >= 0, "gs_reset_opacities: capacity out of range");
  GS_REQUIRE(reset_value > 0.0 && reset_value < 1.0, "gs_reset_opacities: reset value must be in (0, 1)");
  GS_REQUIRE(capacity == 0 || (active && opacities), "gs_reset_opacities: NULL argument");
  if (capacity == 0) return GS_OK;
  // log(p / (1 - p)) of the Python float, rounded once to float32
  const float v = (float)std::log(reset_value / (1.0 - reset_value));
  hipLaunchKernelGGL(reset_opacity_kernel, dim3((unsigned)div_up(capacity, 256)), dim3(256), 0, (hipStream_t)stream,
                     capacity, active, v, opacities);
  GS_LAUNCH_CHECK("reset_opacity_kernel");
  return GS_OK;
}
