// The per-pixel exponent of the compositing kernels and the test that lets a wave skip
// an entry no pixel of its rectangle can blend.  Included by gs_composite.hip (device)
// and by the CPU fuzz test tests/cull_fuzz.cpp (host), so the test checks the very
// expressions the kernels evaluate.
#pragma once

#include <hip/hip_runtime.h>

namespace gs {

// q = log2(e) * power + log2(opacity) with (A, B, C) = log2(e) * (-ic00/2, -ic01,
// -ic11/2), evaluated as (C dy + B dx) dy + (A dx^2 + log2(opacity)); the last term
// and B dx are shared by a lane's pixels.  The forward and backward kernels share
// this exact expression, so they gate the same (pixel, entry) pairs.
__host__ __device__ inline float q_of(float dy, float Adx2l, float Bdx, float C) {
  return fmaf(fmaf(C, dy, Bdx), dy, Adx2l);
}

// True when no point of the rectangle [x0,x1] x [y0,y1] can pass the gate
// power > -10 for the entry (mx, my, A, B, C), where A dx^2 + B dx dy + C dy^2 =
// log2(e) * power.  f = -(A dx^2 + B dx dy + C dy^2) is a convex quadratic when A < 0,
// C < 0 and B^2 < 4AC (anything else, NaN included, is kept); its minimum over the
// rectangle is 0 when the centre lies inside, else it lies on an edge, where it is
// the 1-D minimum at the clamped stationary point.  The threshold exceeds
// 10 log2(e) by an allowance for the rounding of both this minimum and the per-pixel
// exponent (a few ulp of the largest term), so a dropped entry fails the gate at
// every pixel centre of the rectangle as the compositing loops compute it.
__host__ __device__ inline bool entry_misses_rect(float mx, float my, float A, float B, float C, float x0,
                                                  float x1, float y0, float y1) {
  const float a = -A, b = -B, c = -C;
  if (!(a > 0.0f && c > 0.0f && b * b < 4.0f * a * c)) return false;
  const float dx0 = x0 - mx, dx1 = x1 - mx, dy0 = y0 - my, dy1 = y1 - my;
  if (dx0 <= 0.0f && dx1 >= 0.0f && dy0 <= 0.0f && dy1 >= 0.0f) return false;
  const float sx = -0.5f * b / a, sy = -0.5f * b / c;  // stationary points: dx* = sx dy, dy* = sy dx
  auto on_x_edge = [&](float dx) {
    const float dy = fminf(fmaxf(sy * dx, dy0), dy1);
    return (a * dx) * dx + (b * dx) * dy + (c * dy) * dy;
  };
  auto on_y_edge = [&](float dy) {
    const float dx = fminf(fmaxf(sx * dy, dx0), dx1);
    return (a * dx) * dx + (b * dx) * dy + (c * dy) * dy;
  };
  const float fmin = fminf(fminf(on_x_edge(dx0), on_x_edge(dx1)), fminf(on_y_edge(dy0), on_y_edge(dy1)));
  const float ex = fmaxf(dx0 * dx0, dx1 * dx1), ey = fmaxf(dy0 * dy0, dy1 * dy1);
  const float scale = a * ex + fabsf(b) * sqrtf(ex * ey) + c * ey;
  return fmin >= 10.25f * 1.4426950408889634f + 1e-5f * scale;
}

// Exponents at or above this may give exp2(q) >= 0.99, the alpha cap of rasterizer.py:211
// (2^-0.015 = 0.98966: a margin far beyond the rounding of the hardware exp2).
constexpr float kBelowCapQ = -0.015f;

// True when the record (A, B, C, lop) provably keeps q_of below kBelowCapQ at every point
// that passes the gate q > lop - 10 log2(e), wherever the point lies, so that compositing's
// backward may skip the 0.99 cap for it.  With x = (dx, dy), M = [[a, -B/2], [-B/2, c]],
// a = -A, c = -C, the exact form is q* = lop - x^T M x; for M positive definite (eigenvalues
// l1 >= l2 > 0, l1 + l2 = tr, l1 l2 = det) q* <= lop.  q_of's five roundings (A dx, the two
// fmas of the row term, B dx, the last fma) stay within 3u (T + |lop|), u = 2^-24,
// T = |A| dx^2 + |B| |dx dy| + |C| dy^2 <= 2 tr |x|^2.  A gated point has
// x^T M x < 10 log2(e) + err + |lop| u, so with err <= 1, |x|^2 <= 15.5 / l2 <= 15.5 tr / det
// and err <= u (93 tr^2 / det + 3 |lop|).  The test takes u (128 tr^2 / det + 4 |lop| + 4)
// as the bound and asks lop + bound < kBelowCapQ and bound <= 1; every product of two
// floats is exact in double, so det carries one rounding.  NaN or infinite inputs, and
// every matrix that is not positive definite, give false.  Thin Gaussians (tr^2 / det in
// the thousands) and opacities near the cap fail the test and take the per-wave cap test.
__host__ __device__ inline bool record_cannot_cap(float A, float B, float C, float lop) {
  const double a = -(double)A, c = -(double)C, hb = 0.5 * (double)B, l = (double)lop;
  const double det = a * c - hb * hb;
  if (!(a > 0.0 && c > 0.0 && det > 0.0 && l <= 0.0)) return false;
  const double room = (double)kBelowCapQ - l;  // > 0 here
  const double tr = a + c;
  const double lhs = 0x1p-24 * (128.0 * tr * tr + (4.0 * (-l) + 4.0) * det);
  return lhs < (room < 1.0 ? room : 1.0) * det;
}

}  // namespace gs
