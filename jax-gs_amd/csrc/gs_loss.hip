// L1 photometric loss and its gradient seed on gfx950.
// Reference: jax_gs/training/losses.py:4-8, l1_loss(pred, target) = mean(|pred - target|);
// its reverse-mode seed is sign(pred - target) * (1 / count) with sign(0) = 0.
#include "gs_common.h"

namespace gs {
namespace {

__global__ void zero_loss_kernel(float* __restrict__ loss) { loss[0] = 0.0f; }

__global__ __launch_bounds__(256) void l1_kernel(int64_t count, const float* __restrict__ pred,
                                                 const float* __restrict__ target, float inv_count,
                                                 float* __restrict__ loss, float* __restrict__ grad) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  float acc = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const float d = pred[i] - target[i];
    acc += fabsf(d);
    if (grad != nullptr) {
      const float sg = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
      grad[i] = sg * inv_count;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  __shared__ float ws[4];
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(loss, ((ws[0] + ws[1]) + (ws[2] + ws[3])) * inv_count);
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gs_l1_loss(void* stream, int64_t count, const float* pred, const float* target, float* loss,
                          float* grad) {
  GS_REQUIRE(count > 0, "gs_l1_loss: count must be > 0");
  GS_REQUIRE(pred && target && loss, "gs_l1_loss: NULL argument");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(zero_loss_kernel, dim3(1), dim3(1), 0, s, loss);
  GS_LAUNCH_CHECK("zero_loss_kernel");
  const float inv = 1.0f / (float)count;
  int blocks = div_up(count, 256 * 8);
  if (blocks > 2048) blocks = 2048;
  hipLaunchKernelGGL(l1_kernel, dim3(blocks), dim3(256), 0, s, count, pred, target, inv, loss, grad);
  GS_LAUNCH_CHECK("l1_kernel");
  return GS_OK;
}
