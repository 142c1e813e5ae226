// L1 and MSE photometric losses and their gradient seeds on gfx950.
// Reference: jax_gs/training/losses.py:4-8, l1_loss(pred, target) = mean(|pred - target|),
// whose reverse-mode seed is sign(pred - target) * (1 / count) with sign(0) = 0, and
// losses.py:10-14, mse_loss = mean((pred - target)^2), seed 2 (pred - target) / count.
#include "gs_common.h"

#include <algorithm>

namespace gs {
namespace {

__global__ void zero_loss_kernel(float* __restrict__ loss) { loss[0] = 0.0f; }

__device__ inline float sgn(float d) { return d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f); }

// Per-value loss term and gradient seed (before the 1 / count): |d| and sign(d), or
// d^2 and 2 d.
template <bool SQ>
__device__ inline float term(float d) { return SQ ? d * d : fabsf(d); }
template <bool SQ>
__device__ inline float seed(float d) { return SQ ? 2.0f * d : sgn(d); }

// 16-byte loads and stores over the first count/4 quads (when all three arrays are
// 16-byte aligned), scalars for the rest.
template <bool SQ>
__global__ __launch_bounds__(256) void loss_kernel(int64_t count, bool vec, const float* __restrict__ pred,
                                                 const float* __restrict__ target, float inv_count,
                                                 float* __restrict__ loss, float* __restrict__ grad) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nq = vec ? count >> 2 : 0;
  const float4* __restrict__ p4 = reinterpret_cast<const float4*>(pred);
  const float4* __restrict__ t4 = reinterpret_cast<const float4*>(target);
  float4* __restrict__ g4 = reinterpret_cast<float4*>(grad);
  float acc = 0.0f;
#pragma unroll 4
  for (int64_t q = tid; q < nq; q += stride) {
    const float4 a = p4[q], b = t4[q];
    const float d0 = a.x - b.x, d1 = a.y - b.y, d2 = a.z - b.z, d3 = a.w - b.w;
    acc += (term<SQ>(d0) + term<SQ>(d1)) + (term<SQ>(d2) + term<SQ>(d3));
    if (grad != nullptr)
      g4[q] = make_float4(seed<SQ>(d0) * inv_count, seed<SQ>(d1) * inv_count, seed<SQ>(d2) * inv_count,
                          seed<SQ>(d3) * inv_count);
  }
  for (int64_t i = 4 * nq + tid; i < count; i += stride) {
    const float d = pred[i] - target[i];
    acc += term<SQ>(d);
    if (grad != nullptr) grad[i] = seed<SQ>(d) * inv_count;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  __shared__ float ws[4];
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(loss, ((ws[0] + ws[1]) + (ws[2] + ws[3])) * inv_count);
}

// The VJP with the loss cotangent g on the device: grad = seed(d) * (g / count), the
// reference's order (the mean's VJP divides g by the count, the elementwise VJP then
// multiplies by the seed).  One pass: reads both images, writes the gradient.
template <bool SQ>
__global__ __launch_bounds__(256) void loss_bwd_kernel(int64_t count, bool vec, const float* __restrict__ pred,
                                                     const float* __restrict__ target, const float* __restrict__ gout,
                                                     float* __restrict__ grad) {
  const float sc = gout[0] / (float)count;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nq = vec ? count >> 2 : 0;
  const float4* __restrict__ p4 = reinterpret_cast<const float4*>(pred);
  const float4* __restrict__ t4 = reinterpret_cast<const float4*>(target);
  float4* __restrict__ g4 = reinterpret_cast<float4*>(grad);
  for (int64_t q = tid; q < nq; q += stride) {
    const float4 a = p4[q], b = t4[q];
    g4[q] = make_float4(seed<SQ>(a.x - b.x) * sc, seed<SQ>(a.y - b.y) * sc, seed<SQ>(a.z - b.z) * sc,
                        seed<SQ>(a.w - b.w) * sc);
  }
  for (int64_t i = 4 * nq + tid; i < count; i += stride) grad[i] = seed<SQ>(pred[i] - target[i]) * sc;
}

}  // namespace
}  // namespace gs

using namespace gs;

namespace {
template <bool SQ>
int mean_loss(const char* name, void* stream, int64_t count, const float* pred, const float* target, float* loss,
              float* grad) {
  GS_REQUIRE(count > 0, "%s: count must be > 0", name);
  GS_REQUIRE(pred && target && loss, "%s: NULL argument", name);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(zero_loss_kernel, dim3(1), dim3(1), 0, s, loss);
  GS_LAUNCH_CHECK("zero_loss_kernel");
  const float inv = 1.0f / (float)count;
  const bool vec = ((uintptr_t)pred | (uintptr_t)target | (uintptr_t)grad) % 16 == 0;
  // few blocks: each adds its partial sum to loss[0] with one atomic
  int blocks = div_up(count, 256 * 16);
  if (blocks > 512) blocks = 512;
  hipLaunchKernelGGL(loss_kernel<SQ>, dim3(blocks), dim3(256), 0, s, count, vec, pred, target, inv, loss, grad);
  GS_LAUNCH_CHECK("loss_kernel");
  return GS_OK;
}
template <bool SQ>
int mean_loss_bwd(const char* name, void* stream, int64_t count, const float* pred, const float* target,
                  const float* grad_out, float* grad) {
  GS_REQUIRE(count > 0, "%s: count must be > 0", name);
  GS_REQUIRE(pred && target && grad_out && grad, "%s: NULL argument", name);
  const bool vec = ((uintptr_t)pred | (uintptr_t)target | (uintptr_t)grad) % 16 == 0;
  const int blocks = (int)std::min<int64_t>(div_up(vec ? (count + 3) / 4 : count, 256), 8192);
  hipLaunchKernelGGL(loss_bwd_kernel<SQ>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, count, vec, pred, target,
                     grad_out, grad);
  GS_LAUNCH_CHECK("loss_bwd_kernel");
  return GS_OK;
}
}  // namespace

extern "C" int gs_l1_loss_bwd(void* stream, int64_t count, const float* pred, const float* target,
                              const float* grad_out, float* grad) {
  return mean_loss_bwd<false>("gs_l1_loss_bwd", stream, count, pred, target, grad_out, grad);
}

extern "C" int gs_mse_loss_bwd(void* stream, int64_t count, const float* pred, const float* target,
                               const float* grad_out, float* grad) {
  return mean_loss_bwd<true>("gs_mse_loss_bwd", stream, count, pred, target, grad_out, grad);
}

extern "C" int gs_l1_loss(void* stream, int64_t count, const float* pred, const float* target, float* loss,
                          float* grad) {
  return mean_loss<false>("gs_l1_loss", stream, count, pred, target, loss, grad);
}

extern "C" int gs_mse_loss(void* stream, int64_t count, const float* pred, const float* target, float* loss,
                           float* grad) {
  return mean_loss<true>("gs_mse_loss", stream, count, pred, target, loss, grad);
}
