// One masked Adam step of the Gaussian parameter arrays on gfx950.
//
// Reference: train.py:127-155 (optax.multi_transform with one optax.adam per parameter
// array: b1 0.9, b2 0.999, eps 1e-8, eps_root 0), trainer.py:44-53 (_mask_updates:
// rows of inactive Gaussians get a zero update) and optax.apply_updates.  Per element,
// in optax's order of operations (no contraction):
//   mu = (1 - b1) g + b1 mu,   nu = (1 - b2) g^2 + b2 nu,
//   u  = -lr * (mu / (1 - b1^t)) / (sqrt(nu / (1 - b2^t)) + eps),   t = step count + 1,
//   param += active[row] ? u : 0.
// Moments move for every row (the mask applies to the update only, as in the trainer).
//
// The five arrays go in one launch: the grid strides over the concatenation of their
// 4-element chunks, and a chunk's array is found from the chunk offsets.  The row of an
// element (for the mask) is e / row_len by a 64-bit multiply with a precomputed
// reciprocal, exact for e < 2^34 and row_len <= 64.  Pure HBM traffic: 16 B read and
// 12 B written per element.
#include "gs_common.h"

namespace gs {
namespace {

constexpr int kAdamMax = 8;

struct AdamArray {
  float* param;
  const float* grad;
  float* mu;
  float* nu;
  int64_t count;        // elements
  int64_t chunk_begin;  // first 4-element chunk of this array in the launch
  uint64_t row_magic;   // ceil(2^40 / row_len)
  float neg_lr;         // -learning rate
};

struct AdamArgs {
  AdamArray a[kAdamMax];
  int n;
  int64_t chunks;
  float b1, b2, omb1, omb2, bc1, bc2, eps;
};

// floor(e * magic / 2^40) with magic = ceil(2^40 / d): equals e / d for e * (d - 1) < 2^40
__device__ inline int64_t row_of(int64_t e, uint64_t magic) {
  const uint64_t lo = (uint64_t)e * magic, hi = __umul64hi((uint64_t)e, magic);
  return (int64_t)((hi << 24) | (lo >> 40));
}

__device__ inline void adam_elem(const AdamArgs& A, const AdamArray& t, int64_t e, const uint8_t* __restrict__ active,
                                 float g, float& p, float& m, float& v) {
  // optax update_moment / update_moment_per_elem_norm
  m = A.omb1 * g + A.b1 * m;
  v = A.omb2 * (g * g) + A.b2 * v;
  const float u = ((m / A.bc1) / (sqrtf(v / A.bc2) + A.eps)) * t.neg_lr;
  const bool on = active == nullptr || active[row_of(e, t.row_magic)] != 0;
  p = p + (on ? u : 0.0f);
}

__global__ __launch_bounds__(256) void adam_kernel(AdamArgs A, const uint8_t* __restrict__ active) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < A.chunks; c += stride) {
    int k = 0;
#pragma unroll
    for (int j = 1; j < kAdamMax; ++j)
      if (j < A.n && c >= A.a[j].chunk_begin) k = j;
    const AdamArray& t = A.a[k];
    const int64_t e0 = (c - t.chunk_begin) * 4;
    if (e0 + 4 <= t.count && ((reinterpret_cast<uintptr_t>(t.param) | reinterpret_cast<uintptr_t>(t.grad) |
                               reinterpret_cast<uintptr_t>(t.mu) | reinterpret_cast<uintptr_t>(t.nu)) & 15) == 0) {
      float4 p = *reinterpret_cast<const float4*>(t.param + e0);
      const float4 g = *reinterpret_cast<const float4*>(t.grad + e0);
      float4 m = *reinterpret_cast<const float4*>(t.mu + e0);
      float4 v = *reinterpret_cast<const float4*>(t.nu + e0);
      adam_elem(A, t, e0, active, g.x, p.x, m.x, v.x);
      adam_elem(A, t, e0 + 1, active, g.y, p.y, m.y, v.y);
      adam_elem(A, t, e0 + 2, active, g.z, p.z, m.z, v.z);
      adam_elem(A, t, e0 + 3, active, g.w, p.w, m.w, v.w);
      *reinterpret_cast<float4*>(t.param + e0) = p;
      *reinterpret_cast<float4*>(t.mu + e0) = m;
      *reinterpret_cast<float4*>(t.nu + e0) = v;
    } else {
      for (int64_t e = e0; e < e0 + 4 && e < t.count; ++e) {
        float p = t.param[e], m = t.mu[e], v = t.nu[e];
        adam_elem(A, t, e, active, t.grad[e], p, m, v);
        t.param[e] = p;
        t.mu[e] = m;
        t.nu[e] = v;
      }
    }
  }
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gs_adam_step(void* stream, int num_arrays, float* const* params, const float* const* grads,
                            float* const* mus, float* const* nus, const int64_t* counts, const int* row_lens,
                            const double* lrs, const uint8_t* active, int64_t rows, int step, double b1, double b2,
                            double eps) {
  GS_REQUIRE(num_arrays >= 1 && num_arrays <= kAdamMax, "gs_adam_step: 1..%d arrays, got %d", kAdamMax, num_arrays);
  GS_REQUIRE(params && grads && mus && nus && counts && row_lens && lrs, "gs_adam_step: NULL argument");
  GS_REQUIRE(step >= 1, "gs_adam_step: step (count after this update) must be >= 1");
  AdamArgs A{};
  A.n = num_arrays;
  int64_t chunks = 0;
  for (int i = 0; i < num_arrays; ++i) {
    GS_REQUIRE(counts[i] >= 0 && counts[i] < ((int64_t)1 << 34), "gs_adam_step: array %d size %lld", i,
               (long long)counts[i]);
    GS_REQUIRE(row_lens[i] >= 1 && row_lens[i] <= 64, "gs_adam_step: row length of array %d must be 1..64", i);
    GS_REQUIRE(counts[i] == 0 || (params[i] && grads[i] && mus[i] && nus[i]), "gs_adam_step: NULL array %d", i);
    GS_REQUIRE(active == nullptr || counts[i] == rows * row_lens[i],
               "gs_adam_step: array %d has %lld elements, not rows x row length", i, (long long)counts[i]);
    AdamArray& t = A.a[i];
    t.param = params[i];
    t.grad = grads[i];
    t.mu = mus[i];
    t.nu = nus[i];
    t.count = counts[i];
    t.chunk_begin = chunks;
    // ceil(2^40 / row_len): row_of(e) = (e * magic) >> 40
    t.row_magic = (((uint64_t)1 << 40) + (uint64_t)row_lens[i] - 1) / (uint64_t)row_lens[i];
    t.neg_lr = (float)(-lrs[i]);
    chunks += (counts[i] + 3) / 4;
  }
  for (int i = num_arrays; i < kAdamMax; ++i) A.a[i].chunk_begin = chunks;
  A.chunks = chunks;
  // the hyper-parameters are Python floats in the reference: constants formed in double
  // and rounded once to float32, the bias corrections in float32 (optax's jnp.power)
  A.b1 = (float)b1;
  A.b2 = (float)b2;
  A.omb1 = (float)(1.0 - b1);
  A.omb2 = (float)(1.0 - b2);
  A.bc1 = 1.0f - powf((float)b1, (float)step);
  A.bc2 = 1.0f - powf((float)b2, (float)step);
  A.eps = (float)eps;
  if (chunks == 0) return GS_OK;
  hipStream_t s = (hipStream_t)stream;
  // one chunk per thread (measured: 5.5 TB/s at 1M Gaussians, SH3; a grid of 4096
  // looping workgroups reached 4.9)
  const int blocks = (int)std::min<int64_t>(div_up(chunks, 256), (int64_t)1 << 30);
  hipLaunchKernelGGL(adam_kernel, dim3(blocks), dim3(256), 0, s, A, active);
  GS_LAUNCH_CHECK("adam_kernel");
  return GS_OK;
}
