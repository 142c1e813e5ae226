// CPU fuzz of the compositing kernels' entry cull (gs::entry_misses_rect in
// jax-gs_amd/csrc/gs_cull.h) -- test infrastructure, built and run by tests/test_cull.py.
//
// The cull may drop an entry for a wave only if no pixel centre of the wave's rectangle
// passes the gate power > -10, evaluated exactly as the kernels evaluate it:
//   dx = px - mx, Adx2l = fma(A dx, dx, lop), Bdx = B dx,
//   q = q_of(py - my, Adx2l, Bdx, C),  gate: q > thr,  thr = lop - 10 log2(e).
// Records are built as preprocessing writes them (rasterizer.py:147-156: det clamp, inverse,
// scaled by log2(e)).  Two kinds of cases, alternating: (a) the gate's ellipse passes close
// to a random point of the rectangle; (b) the covariance is scaled so that the exact minimum
// over the rectangle of -log2(e) power (in double, each edge minimised in parametric form,
// independently of the cull's own stationary-point formula) lies within 1 % of the cull's
// threshold 10.25 log2(e), so about half of them are dropped and a wrong minimum shows.
// Rectangles are the kernels' three: 16x16 (one wave per tile), 16x8 (two) and 16x4
// (four), at random tiles of a 4096-pixel image.
//
// Output (one line): cases dropped false_drops min_margin
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>

#include "gs_cull.h"

// min over the rectangle of (p - m)^T K (p - m) / 2, K = [[k00, k01], [k01, k11]]
// positive definite, for a centre m outside it: the smallest of the four edges' minima,
// each edge p(t) = a + t (b - a), t in [0, 1].
static double rect_min(double mx, double my, double k00, double k01, double k11, double x0, double x1, double y0,
                       double y1) {
  const double ex[4][4] = {{x0, y0, x1, y0}, {x0, y1, x1, y1}, {x0, y0, x0, y1}, {x1, y0, x1, y1}};
  double best = 1e300;
  for (const auto& e : ex) {
    const double ax = e[0] - mx, ay = e[1] - my, dx = e[2] - e[0], dy = e[3] - e[1];
    const double al = 0.5 * (k00 * dx * dx + 2.0 * k01 * dx * dy + k11 * dy * dy);
    const double be = k00 * ax * dx + k01 * (ax * dy + ay * dx) + k11 * ay * dy;
    const double ga = 0.5 * (k00 * ax * ax + 2.0 * k01 * ax * ay + k11 * ay * ay);
    double t = al > 0.0 ? -be / (2.0 * al) : 0.0;
    t = t < 0.0 ? 0.0 : (t > 1.0 ? 1.0 : t);
    const double v = (al * t + be) * t + ga;
    best = v < best ? v : best;
  }
  return best;
}

int main(int argc, char** argv) {
  const long cases = argc > 1 ? atol(argv[1]) : 1000000;
  const unsigned long long seed = argc > 2 ? strtoull(argv[2], nullptr, 10) : 1ull;
  std::mt19937_64 rng(seed);
  std::uniform_real_distribution<double> U(0.0, 1.0);
  const float L = 1.4426950408889634f;
  long dropped = 0, false_drops = 0;
  double min_margin = 1e30;  // smallest thr - q over the pixels of dropped entries
  for (long t = 0; t < cases; ++t) {
    const int rows = (t % 3 == 0) ? 16 : ((t % 3 == 1) ? 8 : 4);
    const int tx = (int)(U(rng) * 256), ty = (int)(U(rng) * 256);
    const int row0 = rows == 16 ? 0 : rows * (int)(U(rng) * (16 / rows));
    const float x0 = (float)(tx * 16) + 0.5f, x1 = x0 + 15.0f;
    const float y0 = (float)(ty * 16 + row0) + 0.5f, y1 = y0 + (float)(rows - 1);
    // 2-D covariance: eigenvalues log-uniform in [0.3, 3e4] px^2 (the 0.3 low-pass is the
    // floor), random orientation; stored in float32 as projection writes it
    double l1 = 0.3 * std::pow(1e5, U(rng)), l2 = 0.3 * std::pow(1e5, U(rng));
    const double th = U(rng) * 3.141592653589793;
    const double cs = std::cos(th), sn = std::sin(th);
    const bool at_cull = (t & 1) != 0;
    double cmx = 0.0, cmy = 0.0;
    if (at_cull) {
      // a centre outside the rectangle, then the covariance scale that puts the minimum of
      // -power over the rectangle at 10.25 (1 + eps)
      do {
        cmx = x0 - 60.0 + U(rng) * 135.0;
        cmy = y0 - 60.0 + U(rng) * (rows + 119.0);
      } while (cmx >= x0 && cmx <= x1 && cmy >= y0 && cmy <= y1);
      const double i1 = 1.0 / l1, i2 = 1.0 / l2;
      const double k00 = i1 * cs * cs + i2 * sn * sn, k01 = (i1 - i2) * cs * sn, k11 = i1 * sn * sn + i2 * cs * cs;
      const double f0 = rect_min(cmx, cmy, k00, k01, k11, x0, x1, y0, y1);
      const double eps = (U(rng) < 0.3 ? 1e-6 : 0.01) * (2.0 * U(rng) - 1.0);
      const double k = f0 / (10.25 * (1.0 + eps));  // Sigma -> k Sigma divides the form by k
      l1 *= k;
      l2 *= k;
      if (!(l1 > 0.3 && l2 > 0.3 && l1 < 1e7 && l2 < 1e7)) continue;  // outside the covariances projection makes
    }
    const float c00 = (float)(l1 * cs * cs + l2 * sn * sn);
    const float c01 = (float)((l1 - l2) * cs * sn);
    const float c11 = (float)(l1 * sn * sn + l2 * cs * cs);
    const float det = std::fmax(c00 * c11 - c01 * c01, 1e-6f);
    const float ic00 = c11 / det, ic01 = (-c01) / det, ic11 = c00 / det;
    const float A = (-0.5f * ic00) * L, B = (-ic01) * L, C = (-0.5f * ic11) * L;
    const float lop = (float)(-30.0 * U(rng) * U(rng));
    const float thr = lop - 10.0f * L;
    // a target point of the rectangle (often on its border) and a direction; the mean sits
    // so that the gate's boundary along that direction passes within a few percent of it
    double px = x0 - 0.5 + U(rng) * 16.0, py = y0 - 0.5 + U(rng) * rows;
    if (U(rng) < 0.5) {
      if (U(rng) < 0.5) px = U(rng) < 0.5 ? x0 : x1;
      else py = U(rng) < 0.5 ? y0 : y1;
    }
    const double ang = U(rng) * 6.283185307179586;
    const double ux = std::cos(ang), uy = std::sin(ang);
    const double q2 = (double)ic00 * ux * ux + 2.0 * (double)ic01 * ux * uy + (double)ic11 * uy * uy;
    const double s = std::sqrt(20.0 / q2);
    const double eps = (U(rng) < 0.3 ? 1e-6 : 0.05) * (2.0 * U(rng) - 1.0);
    const float mx = at_cull ? (float)cmx : (float)(px - s * (1.0 + eps) * ux);
    const float my = at_cull ? (float)cmy : (float)(py - s * (1.0 + eps) * uy);
    if (!gs::entry_misses_rect(mx, my, A, B, C, x0, x1, y0, y1)) continue;
    ++dropped;
    for (int j = 0; j < rows; ++j) {
      const float pyc = y0 + (float)j;
      for (int i = 0; i < 16; ++i) {
        const float pxc = x0 + (float)i;
        const float dx = pxc - mx;
        const float Adx2l = std::fma(A * dx, dx, lop), Bdx = B * dx;
        const float q = gs::q_of(pyc - my, Adx2l, Bdx, C);
        if (q > thr) ++false_drops;
        const double m = (double)thr - (double)q;
        if (m < min_margin) min_margin = m;
      }
    }
  }
  std::printf("%ld %ld %ld %.9g\n", cases, dropped, false_drops, min_margin);
  return false_drops == 0 ? 0 : 1;
}
