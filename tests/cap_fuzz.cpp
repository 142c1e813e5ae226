// CPU fuzz of the compositing records' cap flag (gs::record_cannot_cap in
// jax-gs_amd/csrc/gs_cull.h, which preprocessing writes into slot 11 of every record) --
// test infrastructure, built and run by tests/test_cull.py.
//
// The backward's four-pixel build skips the 0.99 alpha cap (rasterizer.py:211) for a record
// whose flag is set, so a set flag must mean: at every pixel centre that passes the gate
// q > thr, q < kBelowCapQ, with q evaluated exactly as the kernels evaluate it
//   dx = px - mx, Adx2l = fma(A dx, dx, lop), Bdx = B dx, q = q_of(py - my, Adx2l, Bdx, C).
// Records are built as preprocessing builds them (rasterizer.py:147-156: det clamp, inverse,
// scaled by log2(e)).  Each case puts a 32 x 32 block of pixel centres at a random point of
// the gate's ellipse (anywhere from its centre to its rim, where the exponent's terms are
// largest and cancel most) of a Gaussian at a random sub-pixel position of a 4096-pixel
// image, and evaluates every pixel.
//
// Regimes: "needle" -- one covariance eigenvalue in [1e4, 1e7] px^2, the other in [0.3, 1]
// (long thin Gaussians, where float32 rounding of q reaches whole units), opacities in
// [0.9, 0.995]; "typical" -- both eigenvalues in [0.3, 1e3] px^2, opacities in [0.5, 0.98].
// Rules: "new" is record_cannot_cap; "old" is the rule "op < 0.98 and cov2D positive
// definite", which ignores the rounding (run to show that the fuzz finds its failures).
//
// Output (one line): cases flagged violations min_margin
//   flagged: cases whose flag is set; violations: gated pixels of flagged records with
//   q >= kBelowCapQ; min_margin: smallest kBelowCapQ - q over gated pixels of flagged records.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

#include "gs_cull.h"

int main(int argc, char** argv) {
  const long cases = argc > 1 ? atol(argv[1]) : 100000;
  const unsigned long long seed = argc > 2 ? strtoull(argv[2], nullptr, 10) : 1ull;
  const bool old_rule = argc > 3 && std::strcmp(argv[3], "old") == 0;
  const bool needle = !(argc > 4 && std::strcmp(argv[4], "typical") == 0);
  std::mt19937_64 rng(seed);
  std::uniform_real_distribution<double> U(0.0, 1.0);
  const float L = 1.4426950408889634f;
  long flagged = 0, violations = 0;
  double min_margin = 1e30;
  for (long t = 0; t < cases; ++t) {
    double l1, l2;
    if (needle) {
      l1 = 1e4 * std::pow(1e3, U(rng));
      l2 = 0.3 + 0.7 * U(rng);
    } else {
      l1 = 0.3 * std::pow(1e3 / 0.3, U(rng));
      l2 = 0.3 * std::pow(1e3 / 0.3, U(rng));
    }
    const double th = U(rng) * 3.141592653589793;
    const double cs = std::cos(th), sn = std::sin(th);
    const float c00 = (float)(l1 * cs * cs + l2 * sn * sn);
    const float c01 = (float)((l1 - l2) * cs * sn);
    const float c11 = (float)(l1 * sn * sn + l2 * cs * cs);
    const float det_raw = c00 * c11 - c01 * c01;
    const float det = std::fmax(det_raw, 1e-6f);
    const float ic00 = c11 / det, ic01 = (-c01) / det, ic11 = c00 / det;
    const float A = (-0.5f * ic00) * L, B = (-ic01) * L, C = (-0.5f * ic11) * L;
    const float op = needle ? (float)(0.9 + 0.095 * U(rng)) : (float)(0.5 + 0.48 * U(rng));
    const float lop = std::log2(op);
    const float thr = lop - 10.0f * L;
    const bool flag = old_rule ? (op < 0.98f && det_raw > 0.0f && c00 > 0.0f) : gs::record_cannot_cap(A, B, C, lop);
    if (!flag) continue;
    ++flagged;
    // mean at a random sub-pixel position; the block around a random point of the gate's
    // ellipse x^T Sigma^-1 x < 20 (power > -10), along both axes
    const float mx = (float)(4096.0 * U(rng)), my = (float)(4096.0 * U(rng));
    const double rho = std::sqrt(20.0) * U(rng), phi = U(rng) * 6.283185307179586;
    const double e1 = rho * std::cos(phi) * std::sqrt(l1), e2 = rho * std::sin(phi) * std::sqrt(l2);
    const double cx = mx + e1 * cs - e2 * sn, cy = my + e1 * sn + e2 * cs;
    const double bx = std::floor(cx) - 16.0, by = std::floor(cy) - 16.0;
    for (int j = 0; j < 32; ++j) {
      const float py = (float)(by + j) + 0.5f;
      for (int i = 0; i < 32; ++i) {
        const float px = (float)(bx + i) + 0.5f;
        const float dx = px - mx;
        const float Adx2l = std::fma(A * dx, dx, lop), Bdx = B * dx;
        const float q = gs::q_of(py - my, Adx2l, Bdx, C);
        if (!(q > thr)) continue;
        if (q >= gs::kBelowCapQ) ++violations;
        const double m = (double)gs::kBelowCapQ - (double)q;
        if (m < min_margin) min_margin = m;
      }
    }
  }
  std::printf("%ld %ld %ld %.9g\n", cases, flagged, violations, min_margin);
  return violations == 0 ? 0 : 1;
}
