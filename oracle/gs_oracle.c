/*
 * CPU oracle for the tiled Gaussian-splatting rasterizer -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this
 * library, and only as the checker or the timed CPU baseline; the product path
 * (jax-gs_amd/) never links, loads or calls it.
 *
 * The body (gs_oracle_impl.h) is instantiated in float32 (suffix _f, the restatement
 * the GPU results are compared with) and float64 (suffix _d, used by the tests to
 * check the float restatement and its backward by finite differences).
 *
 * Build (also done by __graft_entry__.build() and oracle/Makefile):
 *   gcc -O2 -std=c99 -fopenmp -ffp-contract=off -fno-fast-math -shared -fPIC gs_oracle.c -o libgsoracle.so -lm
 * -ffp-contract=off keeps every a*b+c as two roundings, as in the reference's
 * float32 expressions evaluated by XLA:CPU without fast-math.
 *
 * Threads (OpenMP): per-Gaussian loops are split over Gaussians, compositing over
 * tiles, the slot sort over contiguous blocks (a stable parallel LSD radix sort).
 * Every output is independent of the thread count except the compositing backward's
 * per-Gaussian sums, which are added per thread and then over the threads in order
 * (the reference's scatter-adds have no specified order either).
 */
#define _GNU_SOURCE
#include <math.h>
#include <omp.h>
#include <sys/mman.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* exp(x) in float32: Cody-Waite reduction x = k ln2 + r with ln2 split into a head
 * with 11 trailing zero bits and a tail, degree-7 Taylor polynomial of e^r by
 * Horner's rule, scaling by 2^k through the exponent field.  Uses only IEEE +,-,*,
 * rint and bit operations, so it returns the same bits as the device-side exp of the
 * product path.  The tests check it against float64 exp (<= 1 ulp). */
float gso_expf(float x) {
  float kf, r, p;
  int k;
  union {
    uint32_t u;
    float f;
  } s;
  if (x > 88.72283f) return HUGE_VALF;
  if (x < -103.97208f) return 0.0f;
  kf = rintf(x * 1.44269504088896341f);
  r = (x - kf * 0.693145751953125f) - kf * 1.42860682030941723212e-6f;
  p = 1.0f / 5040.0f;
  p = p * r + 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  k = (int)kf;
  if (k > 127) {
    p = p * 2.0f;
    k -= 1;
  }
  if (k < -126) {
    p = p * 1.17549435e-38f;
    k += 126;
  }
  s.u = (uint32_t)(k + 127) << 23;
  return p * s.f;
}

/* Large scratch arrays (the 256*n slot keys) on 2 MiB pages: 4 KiB page faults on
 * gigabytes of fresh memory cost more than the sort itself when threads fault in
 * parallel.  gso_hint_huge asks the same for an existing range (the caller's output
 * arrays); both are hints only. */
static void gso_hint_huge(void* p, size_t bytes) {
  const uintptr_t a = ((uintptr_t)p + ((1u << 21) - 1)) & ~(uintptr_t)((1u << 21) - 1);
  const uintptr_t e = ((uintptr_t)p + bytes) & ~(uintptr_t)((1u << 21) - 1);
  if (e > a) madvise((void*)a, e - a, MADV_HUGEPAGE);
}
static void* gso_big_alloc(size_t bytes) {
  void* p = NULL;
  if (posix_memalign(&p, (size_t)1 << 21, bytes ? bytes : 1) != 0) return NULL;
  gso_hint_huge(p, bytes);
  return p;
}

/* gso_expf over an array (vectorised callers in the NumPy layer). */
void gso_expf_array(int64_t n, const float* x, float* y) {
  for (int64_t i = 0; i < n; ++i) y[i] = gso_expf(x[i]);
}

static float gso_sigmoidf(float x) { return 1.0f / (1.0f + gso_expf(-x)); }
static double gso_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

#define REAL float
#define SFX f
#define EXP gso_expf
#define SIGMOID gso_sigmoidf
#define SQRT sqrtf
#define CEIL ceilf
#define FLOOR floorf
#include "gs_oracle_impl.h"
#undef REAL
#undef SFX
#undef EXP
#undef SIGMOID
#undef SQRT
#undef CEIL
#undef FLOOR

#define REAL double
#define SFX d
#define EXP exp
#define SIGMOID gso_sigmoid
#define SQRT sqrt
#define CEIL ceil
#define FLOOR floor
#include "gs_oracle_impl.h"
#undef REAL
#undef SFX
#undef EXP
#undef SIGMOID
#undef SQRT
#undef CEIL
#undef FLOOR

int gso_abi_version(void) { return 3; }

/* Threads used by the parallel loops (0 or less: leave OpenMP's default). */
void gso_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
}
int gso_max_threads(void) { return omp_get_max_threads(); }
