// Per-Gaussian preprocessing on gfx950: EWA projection, 3D/2D covariance, radius,
// SH colour and compositing records (forward), and their vector-Jacobian product
// (backward).  One thread per Gaussian, one wave per 64 Gaussians; every input row
// is read once and every output row written once, so both kernels are HBM-bound.
// Each lane loads its SH row (192 bytes per Gaussian at degree 3) and, backward, its
// gradient record straight into registers with 16-byte loads, which cover the row's
// cache lines whole.
//
// Forward semantics follow, operation by operation and in float32:
//   jax_gs/renderer/projection.py:26-77 (project_gaussians)
//   jax_gs/core/gaussians.py:70-91     (get_covariance_3d)
//   jax_gs/core/camera.py:15-21        (Camera.center)
//   jax_gs/renderer/renderer.py:40-49 + jax_gs/renderer/sh.py:25-72 (colour)
//   jax_gs/renderer/rasterizer.py:147-156 + 198 (conic, sigmoid, 2*ic01)
// The backward is the reverse-mode derivative of that forward with JAX's
// conventions: ties of maximum/minimum/clip split the cotangent 0.5/0.5, the
// radius (ceil) and all masks carry no gradient, and cov2D[1,0] is unused.
#include "gs_common.h"
#include "gs_cull.h"

namespace gs {
namespace {

struct CamRows {
  float w[16];
};

__device__ inline void load_w2c(const float* __restrict__ w2c, float* w) {
#pragma unroll
  for (int k = 0; k < 16; ++k) w[k] = w2c[k];
}

// Quantities of the forward pass that the backward needs again.
struct Proj {
  float x, y, z;            // camera-space mean
  float qn[4], qnorm;       // normalised quaternion (r,x,y,z) and |q|
  float R[3][3], s[3];      // rotation, exp(scales)
  float Mm[3][3];           // R * diag(s)
  float Sig[3][3];          // Mm Mm^T
  float zs, iz, iz2;        // max(z,.01), 1/zs, iz^2
  float M2[2][3];           // J @ W_rot
  float T1[2][3];           // M2 @ Sig
  float c00, c01, c10, c11; // cov2D
};

__device__ inline void project(const float* w, float mx, float my, float mz, const float* q,
                               const float* ls, float fx, float fy, Proj& p) {
  // projection.py:26-29 -- [m,1] @ W2C^T, k ascending.
  p.x = ((mx * w[0] + my * w[1]) + mz * w[2]) + w[3];
  p.y = ((mx * w[4] + my * w[5]) + mz * w[6]) + w[7];
  p.z = ((mx * w[8] + my * w[9]) + mz * w[10]) + w[11];
  // gaussians.py:70-91
  p.qnorm = sqrtf(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
  const float r = q[0] / p.qnorm, x = q[1] / p.qnorm, y = q[2] / p.qnorm, z = q[3] / p.qnorm;
  p.qn[0] = r; p.qn[1] = x; p.qn[2] = y; p.qn[3] = z;
  p.R[0][0] = (1.0f - 2.0f * (y * y)) - 2.0f * (z * z);
  p.R[0][1] = (2.0f * x) * y - (2.0f * r) * z;
  p.R[0][2] = (2.0f * x) * z + (2.0f * r) * y;
  p.R[1][0] = (2.0f * x) * y + (2.0f * r) * z;
  p.R[1][1] = (1.0f - 2.0f * (x * x)) - 2.0f * (z * z);
  p.R[1][2] = (2.0f * y) * z - (2.0f * r) * x;
  p.R[2][0] = (2.0f * x) * z - (2.0f * r) * y;
  p.R[2][1] = (2.0f * y) * z + (2.0f * r) * x;
  p.R[2][2] = (1.0f - 2.0f * (x * x)) - 2.0f * (y * y);
#pragma unroll
  for (int j = 0; j < 3; ++j) p.s[j] = det_expf(ls[j]);
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) p.Mm[i][j] = p.R[i][j] * p.s[j];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      p.Sig[i][j] = (p.Mm[i][0] * p.Mm[j][0] + p.Mm[i][1] * p.Mm[j][1]) + p.Mm[i][2] * p.Mm[j][2];
  // projection.py:43-62
  p.zs = jmax(p.z, 0.01f);
  p.iz = 1.0f / p.zs;
  p.iz2 = p.iz * p.iz;
  const float J[2][3] = {{fx * p.iz, 0.0f, ((-fx) * p.x) * p.iz2},
                         {0.0f, fy * p.iz, ((-fy) * p.y) * p.iz2}};
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      p.M2[i][j] = (J[i][0] * w[0 * 4 + j] + J[i][1] * w[1 * 4 + j]) + J[i][2] * w[2 * 4 + j];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      p.T1[i][j] = (p.M2[i][0] * p.Sig[0][j] + p.M2[i][1] * p.Sig[1][j]) + p.M2[i][2] * p.Sig[2][j];
  float c[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      c[i][j] = (p.T1[i][0] * p.M2[j][0] + p.T1[i][1] * p.M2[j][1]) + p.T1[i][2] * p.M2[j][2];
  const float lp = 0.3f;  // 0.3 * eye(2)
  p.c00 = c[0][0] + lp;
  p.c01 = c[0][1] + 0.0f;
  p.c10 = c[1][0] + 0.0f;
  p.c11 = c[1][1] + lp;
}

// renderer.py:40-41 with camera.py:15-21: unit vector from the camera centre.
__device__ inline void view_dir(const float* w, float mx, float my, float mz, float* v, float& nrm,
                                float* d) {
  float cen[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
    cen[i] = ((-w[0 * 4 + i]) * w[3] + (-w[1 * 4 + i]) * w[7]) + (-w[2 * 4 + i]) * w[11];
  v[0] = mx - cen[0];
  v[1] = my - cen[1];
  v[2] = mz - cen[2];
  nrm = sqrtf((v[0] * v[0] + v[1] * v[1]) + v[2] * v[2]);
  d[0] = v[0] / nrm;
  d[1] = v[1] / nrm;
  d[2] = v[2] / nrm;
}

// sh.py:25-72 for channel c; sh holds coefficient triples (k, channel) at 3k + c.
template <int DEG>
__device__ inline float eval_sh_channel(const float* sh, int c, const float* d) {
  float res = SH_C0 * sh[c];
  if (DEG > 0) {
    const float x = d[0], y = d[1], z = d[2];
    res = ((res - (SH_C1 * y) * sh[3 + c]) + (SH_C1 * z) * sh[6 + c]) - (SH_C1 * x) * sh[9 + c];
    if (DEG > 1) {
      const float xx = x * x, yy = y * y, zz = z * z;
      const float xy = x * y, yz = y * z, xz = x * z;
      res = ((((res + (SH_C2_0 * xy) * sh[12 + c]) + (SH_C2_1 * yz) * sh[15 + c]) +
              (SH_C2_2 * ((2.0f * zz - xx) - yy)) * sh[18 + c]) +
             (SH_C2_3 * xz) * sh[21 + c]) +
            (SH_C2_4 * (xx - yy)) * sh[24 + c];
      if (DEG > 2) {
        res = ((((((res + ((SH_C3_0 * y) * (3.0f * xx - yy)) * sh[27 + c]) +
                   ((SH_C3_1 * xy) * z) * sh[30 + c]) +
                  ((SH_C3_2 * y) * ((4.0f * zz - xx) - yy)) * sh[33 + c]) +
                 ((SH_C3_3 * z) * ((2.0f * zz - 3.0f * xx) - 3.0f * yy)) * sh[36 + c]) +
                ((SH_C3_4 * x) * ((4.0f * zz - xx) - yy)) * sh[39 + c]) +
               ((SH_C3_5 * z) * (xx - yy)) * sh[42 + c]) +
              ((SH_C3_6 * x) * (xx - 3.0f * yy)) * sh[45 + c];
      }
    }
  }
  return res;
}

// rasterizer.py:147-156 and :198 -- record = (mean, -0.5*conic terms, sigmoid, colour),
// and a flag that compositing's backward reads: 1.0 when no pixel that passes the gate
// can reach the 0.99 alpha cap with this record, rounding of the exponent included
// (record_cannot_cap), else 0.0 (the backward then tests the cap per wave).
__device__ inline void write_record(float* __restrict__ rec, float m2x, float m2y, float c00,
                                    float c01, float c11, float logit, const float* col) {
  const float det_raw = c00 * c11 - c01 * c01;
  const float det = jmax(det_raw, 1e-6f);
  const float ic00 = c11 / det;
  const float ic01 = (-c01) / det;
  const float ic11 = c00 / det;
  constexpr float kL2E = 1.4426950408889634f;
  const float op = det_sigmoidf(logit);
  const float lop = log2f(op);
  float4* r4 = reinterpret_cast<float4*>(rec);
  const float A = (-0.5f * ic00) * kL2E, B = (-ic01) * kL2E, C = (-0.5f * ic11) * kL2E;
  r4[0] = make_float4(m2x, m2y, A, B);
  r4[1] = make_float4(C, lop, col[0], col[1]);
  r4[2] = make_float4(col[2], op, lop - 10.0f * kL2E, record_cannot_cap(A, B, C, lop) ? 1.0f : 0.0f);
}

// Copies the first COLS floats of rows [g0, g0+64) of a row-major array (row
// stride `stride` floats) into LDS rows of stride `ls`, consecutive lanes reading
// consecutive addresses (16-byte vectors when rows are 16-byte aligned); every load
// is issued before the first LDS write.  Rows beyond n repeat row n-1 (never used).
template <int COLS>
__device__ inline void stage_rows(const float* __restrict__ src, int64_t g0, int64_t n, int64_t stride,
                                  float* __restrict__ lds, int ls, int lane) {
  constexpr int C4 = COLS / 4 > 0 ? COLS / 4 : 1;
  const float* __restrict__ base = src + g0 * stride;
  const int rmax = (int)(n - 1 - g0 < 63 ? n - 1 - g0 : 63);
  const uint32_t st = (uint32_t)stride;
  if ((COLS & 3) == 0 && (stride & 3) == 0) {
    float4 v[C4];
#pragma unroll
    for (int t = 0; t < C4; ++t) {
      const int e = lane + 64 * t, r = e / C4, c = e - r * C4;
      const uint32_t off = (uint32_t)min(r, rmax) * st + 4u * (uint32_t)c;
      v[t] = *reinterpret_cast<const float4*>(base + off);
    }
#pragma unroll
    for (int t = 0; t < C4; ++t) {
      const int e = lane + 64 * t, r = e / C4, c = e - r * C4;
      float* d = lds + r * ls + 4 * c;
      d[0] = v[t].x;
      d[1] = v[t].y;
      d[2] = v[t].z;
      d[3] = v[t].w;
    }
  } else {
#pragma unroll 8
    for (int t = 0; t < COLS; ++t) {
      const int e = lane + 64 * t, r = e / COLS, c = e - r * COLS;
      lds[r * ls + c] = base[(uint32_t)min(r, rmax) * st + (uint32_t)c];
    }
  }
}

// The first COLS floats of one row into registers: 16-byte loads when the row is
// 16-byte aligned.
template <int COLS>
__device__ inline void load_row(const float* __restrict__ row, bool aligned, float* __restrict__ out) {
  if ((COLS & 3) == 0 && aligned) {
#pragma unroll
    for (int t = 0; t < COLS / 4; ++t) {
      const float4 v = reinterpret_cast<const float4*>(row)[t];
      out[4 * t] = v.x;
      out[4 * t + 1] = v.y;
      out[4 * t + 2] = v.z;
      out[4 * t + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int t = 0; t < COLS; ++t) out[t] = row[t];
  }
}

// One thread per Gaussian, one wave per 64 Gaussians.  Each lane loads its own SH row
// (3 (D+1)^2 floats) straight into registers: with no LDS staging buffer the kernel
// holds 6 waves per SIMD instead of 3 (LDS-bound), which measured faster at 1080p SH3
// than coalesced staging through LDS (every row's cache lines are still read whole by
// the wave's 16-byte loads).
template <int DEG>
__global__ __launch_bounds__(64) void preprocess_fwd_kernel(
    int64_t n, int K, const float* __restrict__ means, const float* __restrict__ scales,
    const float* __restrict__ quats, const float* __restrict__ opac, const float* __restrict__ sh,
    const uint8_t* __restrict__ mask, const float* __restrict__ w2c, float fx, float fy, float cx,
    float cy, float* __restrict__ means2d, float* __restrict__ cov2d, float* __restrict__ radii,
    uint8_t* __restrict__ valid, float* __restrict__ depths, float* __restrict__ colors,
    float* __restrict__ records) {
  constexpr int NB = (DEG + 1) * (DEG + 1);
  const int lane = threadIdx.x;
  const int64_t g0 = (int64_t)blockIdx.x * 64;
  const int64_t i = g0 + lane;
  // per-Gaussian inputs first (clamped index), so that their loads are in flight
  // together with the SH row's
  const int64_t ic = i < n ? i : n - 1;
  const float mx = means[3 * ic], my = means[3 * ic + 1], mz = means[3 * ic + 2];
  float q[4], ls[3];
#pragma unroll
  for (int k = 0; k < 4; ++k) q[k] = quats[4 * ic + k];
#pragma unroll
  for (int k = 0; k < 3; ++k) ls[k] = scales[3 * ic + k];
  const float logit = opac[ic];
  // A masked-out Gaussian is never an entry, so no compositing reads its record's colour:
  // without a colour output its SH row is not read (the record's colour is then that of
  // zero coefficients).  Without a mask nothing waits for the mask byte.
  const bool sh_needed = colors != nullptr || mask == nullptr || mask[ic] != 0;
  float shv[3 * NB];
  if (sh_needed) {
    load_row<3 * NB>(sh + ic * (int64_t)(3 * K), (3 * K) % 4 == 0, shv);
  } else {
#pragma unroll
    for (int k = 0; k < 3 * NB; ++k) shv[k] = 0.0f;
  }
  if (i >= n) return;
  float w[16];
  load_w2c(w2c, w);
  Proj p;
  project(w, mx, my, mz, q, ls, fx, fy, p);
  const bool v = (p.z > 0.01f) && (mask == nullptr || mask[i] != 0);
  // projection.py:65-68 -- raw z here.
  const float m2x = (fx * p.x) / p.z + cx;
  const float m2y = (fy * p.y) / p.z + cy;
  // projection.py:71-77
  const float det = p.c00 * p.c11 - p.c01 * p.c01;
  const float mid = (p.c00 + p.c11) / 2.0f;
  const float term = sqrtf(jmax(mid * mid - det, 0.0f));
  const float radius = ceilf(3.0f * sqrtf(mid + term));
  // renderer.py:40-49
  float vv[3], nrm, d[3];
  view_dir(w, mx, my, mz, vv, nrm, d);
  float col[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float res = eval_sh_channel<DEG>(shv, c, d) + 0.5f;
    col[c] = jmin(1.0f, jmax(0.0f, res));
  }
  means2d[2 * i] = m2x;
  means2d[2 * i + 1] = m2y;
  if (cov2d != nullptr) reinterpret_cast<float4*>(cov2d)[i] = make_float4(p.c00, p.c01, p.c10, p.c11);
  radii[i] = radius;
  valid[i] = v ? 1 : 0;
  depths[i] = p.z;
  if (colors != nullptr) {
    colors[3 * i] = col[0];
    colors[3 * i + 1] = col[1];
    colors[3 * i + 2] = col[2];
  }
  if (records != nullptr) write_record(records + i * kRec, m2x, m2y, p.c00, p.c01, p.c11, logit, col);
}

__global__ __launch_bounds__(256) void composite_prep_kernel(int64_t n, const float* __restrict__ means2d,
                                                             const float* __restrict__ cov2d,
                                                             const float* __restrict__ opac,
                                                             const float* __restrict__ colors,
                                                             float* __restrict__ records) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float4 c = reinterpret_cast<const float4*>(cov2d)[i];
  const float col[3] = {colors[3 * i], colors[3 * i + 1], colors[3 * i + 2]};
  write_record(records + i * kRec, means2d[2 * i], means2d[2 * i + 1], c.x, c.y, c.w, opac[i], col);
}

// eval_sh_channel's factors F[k], rounded as it rounds them: colour c is
// F[0] s0 - F[1] s1 + F[2] s2 - F[3] s3 + F[4] s4 + ... (k = 1 and 3 subtract).
template <int DEG>
__device__ inline void sh_factors(const float* d, float* F) {
  const float x = d[0], y = d[1], z = d[2];
  const float xx = x * x, yy = y * y, zz = z * z;
  const float xy = x * y, yz = y * z, xz = x * z;
  F[0] = SH_C0;
  if (DEG > 0) {
    F[1] = SH_C1 * y;
    F[2] = SH_C1 * z;
    F[3] = SH_C1 * x;
  }
  if (DEG > 1) {
    F[4] = SH_C2_0 * xy;
    F[5] = SH_C2_1 * yz;
    F[6] = SH_C2_2 * ((2.0f * zz - xx) - yy);
    F[7] = SH_C2_3 * xz;
    F[8] = SH_C2_4 * (xx - yy);
  }
  if (DEG > 2) {
    F[9] = (SH_C3_0 * y) * (3.0f * xx - yy);
    F[10] = (SH_C3_1 * xy) * z;
    F[11] = (SH_C3_2 * y) * ((4.0f * zz - xx) - yy);
    F[12] = (SH_C3_3 * z) * ((2.0f * zz - 3.0f * xx) - 3.0f * yy);
    F[13] = (SH_C3_4 * x) * ((4.0f * zz - xx) - yy);
    F[14] = (SH_C3_5 * z) * (xx - yy);
    F[15] = (SH_C3_6 * x) * (xx - 3.0f * yy);
  }
}

// basis_k and d basis_k / d(x,y,z) of the degree<=3 real SH basis of eval_sh_channel.
template <int DEG>
__device__ inline void sh_basis_and_grad(const float* d, float* B, float (*dB)[3]) {
  constexpr int deg = DEG;
  const float x = d[0], y = d[1], z = d[2];
  const float xx = x * x, yy = y * y, zz = z * z;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    B[k] = 0.0f;
    dB[k][0] = dB[k][1] = dB[k][2] = 0.0f;
  }
  B[0] = SH_C0;
  if (deg > 0) {
    B[1] = -SH_C1 * y; dB[1][1] = -SH_C1;
    B[2] = SH_C1 * z;  dB[2][2] = SH_C1;
    B[3] = -SH_C1 * x; dB[3][0] = -SH_C1;
  }
  if (deg > 1) {
    B[4] = SH_C2_0 * x * y; dB[4][0] = SH_C2_0 * y; dB[4][1] = SH_C2_0 * x;
    B[5] = SH_C2_1 * y * z; dB[5][1] = SH_C2_1 * z; dB[5][2] = SH_C2_1 * y;
    B[6] = SH_C2_2 * (2.0f * zz - xx - yy);
    dB[6][0] = SH_C2_2 * (-2.0f * x); dB[6][1] = SH_C2_2 * (-2.0f * y); dB[6][2] = SH_C2_2 * (4.0f * z);
    B[7] = SH_C2_3 * x * z; dB[7][0] = SH_C2_3 * z; dB[7][2] = SH_C2_3 * x;
    B[8] = SH_C2_4 * (xx - yy); dB[8][0] = SH_C2_4 * (2.0f * x); dB[8][1] = SH_C2_4 * (-2.0f * y);
  }
  if (deg > 2) {
    B[9] = SH_C3_0 * y * (3.0f * xx - yy);
    dB[9][0] = SH_C3_0 * (6.0f * x * y); dB[9][1] = SH_C3_0 * (3.0f * xx - 3.0f * yy);
    B[10] = SH_C3_1 * x * y * z;
    dB[10][0] = SH_C3_1 * y * z; dB[10][1] = SH_C3_1 * x * z; dB[10][2] = SH_C3_1 * x * y;
    B[11] = SH_C3_2 * y * (4.0f * zz - xx - yy);
    dB[11][0] = SH_C3_2 * (-2.0f * x * y); dB[11][1] = SH_C3_2 * (4.0f * zz - xx - 3.0f * yy);
    dB[11][2] = SH_C3_2 * (8.0f * y * z);
    B[12] = SH_C3_3 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
    dB[12][0] = SH_C3_3 * (-6.0f * x * z); dB[12][1] = SH_C3_3 * (-6.0f * y * z);
    dB[12][2] = SH_C3_3 * (6.0f * zz - 3.0f * xx - 3.0f * yy);
    B[13] = SH_C3_4 * x * (4.0f * zz - xx - yy);
    dB[13][0] = SH_C3_4 * (4.0f * zz - 3.0f * xx - yy); dB[13][1] = SH_C3_4 * (-2.0f * x * y);
    dB[13][2] = SH_C3_4 * (8.0f * x * z);
    B[14] = SH_C3_5 * z * (xx - yy);
    dB[14][0] = SH_C3_5 * (2.0f * x * z); dB[14][1] = SH_C3_5 * (-2.0f * y * z); dB[14][2] = SH_C3_5 * (xx - yy);
    B[15] = SH_C3_6 * x * (xx - 3.0f * yy);
    dB[15][0] = SH_C3_6 * (3.0f * xx - 3.0f * yy); dB[15][1] = SH_C3_6 * (-6.0f * x * y);
  }
}

struct GaussIn {
  float mx, my, mz, q[4], ls[3], logit;
};

__device__ inline GaussIn load_gauss(const float* __restrict__ means, const float* __restrict__ scales,
                                     const float* __restrict__ quats, const float* __restrict__ opac, int64_t i) {
  GaussIn a;
  a.mx = means[3 * i];
  a.my = means[3 * i + 1];
  a.mz = means[3 * i + 2];
#pragma unroll
  for (int k = 0; k < 4; ++k) a.q[k] = quats[4 * i + k];
#pragma unroll
  for (int k = 0; k < 3; ++k) a.ls[k] = scales[3 * i + k];
  a.logit = opac[i];
  return a;
}

// The colour VJP of one Gaussian (renderer.py:40-49 and sh.py:25-72, reversed).  One pass
// over the SH row forms the three colours from eval_sh_channel's terms in its order (so the
// clip mask is the forward's, bit for bit) together with the nine partials
// V[c] = sum_k sh[k][c] dbasis_k/dd; the row is dead afterwards.  Outputs: E[k], the
// signed basis value multiplying coefficient k in that sum (the SH cotangent row is
// E[k] * g_pre[c]), g_pre[c] = dL/d(colour before the clip), and the mean's cotangent
// through the view direction, added to g_m.
template <int DEG>
__device__ inline void colour_vjp(const float* w, float mx, float my, float mz, const float* shv, const float* g_col,
                                  float* E, float* g_pre, float* g_m) {
  constexpr int NB = (DEG + 1) * (DEG + 1);
  float vv[3], nrm, d[3];
  view_dir(w, mx, my, mz, vv, nrm, d);
  // eval_sh_channel's factors; k = 1 and 3 enter with a minus sign
  float F[16];
  sh_factors<DEG>(d, F);
  float B[16], dB[16][3];
  sh_basis_and_grad<DEG>(d, B, dB);  // (only the derivatives are used)
  float res[3], V[3][3];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    res[c] = F[0] * shv[c];
    V[c][0] = V[c][1] = V[c][2] = 0.0f;
  }
#pragma unroll
  for (int k = 1; k < NB; ++k) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float sk = shv[3 * k + c];
      res[c] = (k == 1 || k == 3) ? res[c] - F[k] * sk : res[c] + F[k] * sk;
      V[c][0] += sk * dB[k][0];
      V[c][1] += sk * dB[k][1];
      V[c][2] += sk * dB[k][2];
    }
  }
#pragma unroll
  for (int k = 0; k < NB; ++k) E[k] = (k == 1 || k == 3) ? -F[k] : F[k];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float pre = res[c] + 0.5f;
    const float lo = jmax(0.0f, pre);
    g_pre[c] = g_col[c] * dmin_first(lo, 1.0f) * dmax_first(pre, 0.0f);
  }
  if (DEG > 0) {
    float g_d[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) g_d[j] = (g_pre[0] * V[0][j] + g_pre[1] * V[1][j]) + g_pre[2] * V[2][j];
    const float dg = (d[0] * g_d[0] + d[1] * g_d[1]) + d[2] * g_d[2];
#pragma unroll
    for (int k = 0; k < 3; ++k) g_m[k] += (g_d[k] - d[k] * dg) / nrm;
  }
}

// The conic and opacity part of the backward (rasterizer.py:147-156 reversed): from a
// Gaussian's gradient record grow and its cov2D (c00, c01, c11) and opacity logit, the
// cotangents of means2D, of cov2D (G; render_tiles never reads cov2D[1,0], so G[1][0] = 0)
// and of the logit.
__device__ inline void conic_vjp(const float* grow, float c00, float c01, float c11, float logit, float& g_m2x,
                                 float& g_m2y, float (&G)[2][2], float& g_logit) {
  const float4 ga = make_float4(grow[0], grow[1], grow[2], grow[3]);
  const float4 gb = make_float4(grow[4], grow[5], grow[6], grow[7]);
  // gradient record (sums over the Gaussian's pixels of dL/dpower times):
  // [0] dx, [1] dy, [2] dx^2, [3] dx dy, [4] dy^2, [5] 1; [6..8] dL/dcolour
  // power = -0.5 (ic00 dx^2 + 2 ic01 dx dy + ic11 dy^2), dx = px - mean2d.x
  const float g_ic00 = -0.5f * ga.z;
  const float g_ic01 = -ga.w;
  const float g_ic11 = -0.5f * gb.x;

  // ---- opacity: alpha = exp(power) * sigmoid(logit); sum dL/dpower = sigmoid * dL/dsigmoid
  const float sg = det_sigmoidf(logit);
  g_logit = gb.y * (1.0f - sg);

  // ---- conic <- cov2D (rasterizer.py:147-153)
  const float det_raw = c00 * c11 - c01 * c01;
  const float det = jmax(det_raw, 1e-6f);
  const float ic00 = c11 / det, ic01 = (-c01) / det, ic11 = c00 / det;
  // ---- d power / d mean2d = (ic00 dx + ic01 dy, ic01 dx + ic11 dy)
  g_m2x = ic00 * ga.x + ic01 * ga.y;
  g_m2y = ic01 * ga.x + ic11 * ga.y;
  float g_c00 = g_ic11 / det;
  float g_c11 = g_ic00 / det;
  float g_c01 = -g_ic01 / det;
  const float g_det = -((g_ic00 * ic00 + g_ic01 * ic01) + g_ic11 * ic11) / det * dmax_first(det_raw, 1e-6f);
  g_c00 += g_det * c11;
  g_c11 += g_det * c00;
  g_c01 += -2.0f * c01 * g_det;
  G[0][0] = g_c00;
  G[0][1] = g_c01;
  G[1][0] = 0.0f;
  G[1][1] = g_c11;
}

// The projection part of the backward of one Gaussian (project_gaussians and
// get_covariance_3d reversed, projection.py:26-79, gaussians.py:58-92): from the
// cotangents of means2D (g_m2x, g_m2y), cov2D (G, all four entries) and, with DEPTH, of
// the depth z (g_depth), to those of the mean, log-scales and quaternion.  p is the
// Gaussian's forward projection.  g_mcol: the mean's cotangent through the view direction
// (colour_vjp), added last.  part (may be NULL): the Gaussian's share of dL/dW2C through
// the camera-space mean and W_rot, part[3a+b] for W2C[a][b] and part[9+a] for W2C[a][3]
// (projection.py:26-27, 52-57).
template <bool DEPTH>
__device__ inline void project_vjp(int64_t i, const GaussIn& in, const Proj& p, const float* w, float fx, float fy,
                                   float g_m2x, float g_m2y, const float (&G)[2][2], float g_depth,
                                   const float* g_mcol, float* __restrict__ g_means, float* __restrict__ g_scales,
                                   float* __restrict__ g_quats, float* part) {
  const float mx = in.mx, my = in.my, mz = in.mz;
  // ---- cov2D = (M2 Sig) M2^T + 0.3 I
  float g_T1[2][3], g_M2[2][3], g_Sig[3][3];
#pragma unroll
  for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      g_T1[i2][j] = G[i2][0] * p.M2[0][j] + G[i2][1] * p.M2[1][j];
      g_M2[i2][j] = G[0][i2] * p.T1[0][j] + G[1][i2] * p.T1[1][j];
    }
#pragma unroll
  for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      g_M2[i2][j] += (g_T1[i2][0] * p.Sig[j][0] + g_T1[i2][1] * p.Sig[j][1]) + g_T1[i2][2] * p.Sig[j][2];
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 3; ++j) g_Sig[k][j] = p.M2[0][k] * g_T1[0][j] + p.M2[1][k] * g_T1[1][j];

  // ---- M2 = J W_rot
  float g_J[2][3];
#pragma unroll
  for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
    for (int k = 0; k < 3; ++k)
      g_J[i2][k] = (g_M2[i2][0] * w[k * 4 + 0] + g_M2[i2][1] * w[k * 4 + 1]) + g_M2[i2][2] * w[k * 4 + 2];
  float g_x = 0.0f, g_y = 0.0f, g_z = 0.0f;
  float g_iz = fx * g_J[0][0] + fy * g_J[1][1];
  const float g_iz2 = ((-fx) * p.x) * g_J[0][2] + ((-fy) * p.y) * g_J[1][2];
  g_x += (-fx) * p.iz2 * g_J[0][2];
  g_y += (-fy) * p.iz2 * g_J[1][2];
  g_iz += 2.0f * p.iz * g_iz2;
  const float g_zs = -g_iz * p.iz * p.iz;
  g_z += g_zs * dmax_first(p.z, 0.01f);
  // ---- means2D = f*x/z + c (raw z)
  g_x += g_m2x * fx / p.z;
  g_y += g_m2y * fy / p.z;
  g_z += -(g_m2x * (fx * p.x) + g_m2y * (fy * p.y)) / (p.z * p.z);
  // ---- z itself (project_gaussians returns it)
  if (DEPTH) g_z += g_depth;
  if (part != nullptr) {
    // means_cam = W_rot m + t;  M2 = J W_rot with J = [[fx iz, 0, -fx x iz2], [0, fy iz, -fy y iz2]]
    const float J0[3] = {fx * p.iz, 0.0f, ((-fx) * p.x) * p.iz2};
    const float J1[3] = {0.0f, fy * p.iz, ((-fy) * p.y) * p.iz2};
    const float gp[3] = {g_x, g_y, g_z}, m[3] = {mx, my, mz};
#pragma unroll
    for (int a = 0; a < 3; ++a) {
#pragma unroll
      for (int b = 0; b < 3; ++b) part[3 * a + b] = gp[a] * m[b] + (J0[a] * g_M2[0][b] + J1[a] * g_M2[1][b]);
      part[9 + a] = gp[a];
    }
  }
  // ---- camera-space mean <- world mean
  float g_m[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) g_m[k] = (w[0 * 4 + k] * g_x + w[1 * 4 + k] * g_y) + w[2 * 4 + k] * g_z;

  // ---- the colour's share through the view direction (colour_vjp)
#pragma unroll
  for (int k = 0; k < 3; ++k) g_m[k] += g_mcol[k];
  g_means[3 * i] = g_m[0];
  g_means[3 * i + 1] = g_m[1];
  g_means[3 * i + 2] = g_m[2];

  // ---- Sig = Mm Mm^T, Mm = R diag(s), s = exp(ls)
  float g_Mm[3][3];
#pragma unroll
  for (int a = 0; a < 3; ++a)
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 3; ++k) acc += (g_Sig[a][k] + g_Sig[k][a]) * p.Mm[k][b];
      g_Mm[a][b] = acc;
    }
  float g_R[3][3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    float gs = 0.0f;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      g_R[a][j] = g_Mm[a][j] * p.s[j];
      gs += g_Mm[a][j] * p.R[a][j];
    }
    g_scales[3 * i + j] = gs * p.s[j];
  }
  // ---- R(qn)
  const float r = p.qn[0], x = p.qn[1], y = p.qn[2], z = p.qn[3];
  float gr = 0.0f, gx = 0.0f, gy = 0.0f, gz = 0.0f;
  gy += -4.0f * y * g_R[0][0]; gz += -4.0f * z * g_R[0][0];
  gx += 2.0f * y * g_R[0][1]; gy += 2.0f * x * g_R[0][1]; gr += -2.0f * z * g_R[0][1]; gz += -2.0f * r * g_R[0][1];
  gx += 2.0f * z * g_R[0][2]; gz += 2.0f * x * g_R[0][2]; gr += 2.0f * y * g_R[0][2]; gy += 2.0f * r * g_R[0][2];
  gx += 2.0f * y * g_R[1][0]; gy += 2.0f * x * g_R[1][0]; gr += 2.0f * z * g_R[1][0]; gz += 2.0f * r * g_R[1][0];
  gx += -4.0f * x * g_R[1][1]; gz += -4.0f * z * g_R[1][1];
  gy += 2.0f * z * g_R[1][2]; gz += 2.0f * y * g_R[1][2]; gr += -2.0f * x * g_R[1][2]; gx += -2.0f * r * g_R[1][2];
  gx += 2.0f * z * g_R[2][0]; gz += 2.0f * x * g_R[2][0]; gr += -2.0f * y * g_R[2][0]; gy += -2.0f * r * g_R[2][0];
  gy += 2.0f * z * g_R[2][1]; gz += 2.0f * y * g_R[2][1]; gr += 2.0f * x * g_R[2][1]; gx += 2.0f * r * g_R[2][1];
  gx += -4.0f * x * g_R[2][2]; gy += -4.0f * y * g_R[2][2];
  // ---- qn = q / |q|
  const float gq[4] = {gr, gx, gy, gz};
  const float qd = ((p.qn[0] * gq[0] + p.qn[1] * gq[1]) + p.qn[2] * gq[2]) + p.qn[3] * gq[3];
#pragma unroll
  for (int k = 0; k < 4; ++k) g_quats[4 * i + k] = (gq[k] - p.qn[k] * qd) / p.qnorm;
}

// Geometric part of the backward of one Gaussian from its gradient record grow (conic,
// opacity, projection, covariance); g_mcol and part as for project_vjp.
__device__ inline void preprocess_bwd_geom(int64_t i, const GaussIn& in, const float* w, float fx, float fy,
                                           const float* grow, const float* g_mcol, float* __restrict__ g_means,
                                           float* __restrict__ g_scales, float* __restrict__ g_quats,
                                           float* __restrict__ g_opac, float* part = nullptr) {
  float q[4], ls[3];
#pragma unroll
  for (int k = 0; k < 4; ++k) q[k] = in.q[k];
#pragma unroll
  for (int k = 0; k < 3; ++k) ls[k] = in.ls[k];
  Proj p;
  project(w, in.mx, in.my, in.mz, q, ls, fx, fy, p);
  float g_m2x, g_m2y, G[2][2], g_logit;
  conic_vjp(grow, p.c00, p.c01, p.c11, in.logit, g_m2x, g_m2y, G, g_logit);
  g_opac[i] = g_logit;
  project_vjp<false>(i, in, p, w, fx, fy, g_m2x, g_m2y, G, 0.0f, g_mcol, g_means, g_scales, g_quats, part);
}

// Backward of one Gaussian.  shv: its SH row (registers), overwritten with the SH
// cotangent row (K triples, coefficients >= (D+1)^2 get 0); grow: its gradient record.
template <int DEG>
__device__ inline void preprocess_bwd_one(int64_t i, int K, const GaussIn& in, const float* __restrict__ w2c,
                                          float fx, float fy, const float* grow, float* shv,
                                          float* __restrict__ g_means, float* __restrict__ g_scales,
                                          float* __restrict__ g_quats, float* __restrict__ g_opac) {
  constexpr int NB = (DEG + 1) * (DEG + 1);
  float w[16];
  load_w2c(w2c, w);
  float E[16], g_pre[3], g_mcol[3] = {0.0f, 0.0f, 0.0f};
  const float g_col[3] = {grow[6], grow[7], grow[8]};
  colour_vjp<DEG>(w, in.mx, in.my, in.mz, shv, g_col, E, g_pre, g_mcol);
#pragma unroll
  for (int k = 0; k < NB; ++k)
#pragma unroll
    for (int c = 0; c < 3; ++c) shv[3 * k + c] = E[k] * g_pre[c];
  for (int q = 3 * NB; q < 3 * K; ++q) shv[q] = 0.0f;
  preprocess_bwd_geom(i, in, w, fx, fy, grow, g_mcol, g_means, g_scales, g_quats, g_opac);
}

// Sum over the wave's 64 lanes (every lane gets it).
__device__ inline float wave_total(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// The backward of Gaussian i from its inputs, SH row shv and gradient record grow;
// part (may be NULL): its share of dL/dW2C (preprocess_bwd_geom's 12 values and the view
// vector's cotangent in part[12..14]).
template <int DEG>
__device__ inline void preprocess_bwd_gauss(int64_t i, int K, const GaussIn& in, const float* __restrict__ w2c,
                                            float fx, float fy, const float* shv, const float* grow, bool aligned,
                                            float* __restrict__ g_means, float* __restrict__ g_scales,
                                            float* __restrict__ g_quats, float* __restrict__ g_opac,
                                            float* __restrict__ g_sh, float* part) {
  constexpr int NB = (DEG + 1) * (DEG + 1);
  const int KC = 3 * K;
  float w[16];
  load_w2c(w2c, w);
  // the colour VJP first: the SH row is dead once it returns, so the geometric VJP
  // below does not hold it
  float E[16], g_pre[3], g_mcol[3] = {0.0f, 0.0f, 0.0f};
  const float g_col[3] = {grow[6], grow[7], grow[8]};
  colour_vjp<DEG>(w, in.mx, in.my, in.mz, shv, g_col, E, g_pre, g_mcol);
  float* __restrict__ dst = g_sh + i * KC;
  auto cot = [&](int t) { return t < 3 * NB ? E[t / 3] * g_pre[t % 3] : 0.0f; };
  if (aligned && (3 * NB) % 4 == 0) {
#pragma unroll
    for (int t = 0; t < 3 * NB / 4; ++t)
      reinterpret_cast<float4*>(dst)[t] = make_float4(cot(4 * t), cot(4 * t + 1), cot(4 * t + 2), cot(4 * t + 3));
    for (int t = 3 * NB / 4; t < KC / 4; ++t) reinterpret_cast<float4*>(dst)[t] = make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
#pragma unroll
    for (int t = 0; t < 3 * NB; ++t) dst[t] = cot(t);
    for (int t = 3 * NB; t < KC; ++t) dst[t] = 0.0f;
  }
  preprocess_bwd_geom(i, in, w, fx, fy, grow, g_mcol, g_means, g_scales, g_quats, g_opac, part);
  if (part != nullptr) {
#pragma unroll
    for (int k = 0; k < 3; ++k) part[12 + k] = g_mcol[k];
  }
}

// Zero cotangents of Gaussian i's five arrays (KC = 3 K floats of SH).
// Zeros floats [begin, end) of p with the block's threads (NT of them), consecutive threads on
// consecutive 16-byte words: scalar stores up to the first 16-byte boundary and after the last.
template <int NT>
__device__ inline void zero_block(float* __restrict__ p, int64_t begin, int64_t end, int t) {
  if (begin >= end) return;
  int64_t a = begin;
  while (a < end && ((reinterpret_cast<uintptr_t>(p + a) & 15) != 0)) ++a;  // <= 3 floats
  const int64_t nv = (end - a) / 4;
  if (t < a - begin) p[begin + t] = 0.0f;
  typedef float f4v __attribute__((ext_vector_type(4)));
  f4v* __restrict__ v = reinterpret_cast<f4v*>(p + a);
  const f4v z = {0.f, 0.f, 0.f, 0.f};
  for (int64_t j = t; j < nv; j += NT) __builtin_nontemporal_store(z, v + j);
  const int64_t tail = a + 4 * nv;
  if (t < end - tail) p[tail + t] = 0.0f;
}

// The preprocessing VJP.  A Gaussian that no pixel's cotangent reached (off-screen, masked,
// or occluded -- in a dense scene most are: 96 % of configuration 2's million, 77 % of
// configuration 1's) has an all-zero gradient record, and its VJP is then exactly zero
// (every term is a product with a record value; the parameters only need to be finite).
// A workgroup takes SPAN consecutive Gaussians: its threads read the span's records, zero the
// span's gradient rows (coalesced; no parameter or SH row is read for it) and list the reached
// Gaussians in LDS; the list is then processed one Gaussian per thread, so
// the arithmetic runs in full waves of reached Gaussians (with one thread per Gaussian
// every wave holding a reached one would run it whole).  A reached Gaussian's SH row and
// gradient record are loaded straight into registers and its SH cotangent row stored from
// them (16-byte accesses when rows are 16-byte aligned).
// W2C: each workgroup also writes its reached Gaussians' summed shares of dL/dW2C (15
// floats: through the mean and W_rot, then the view vector's cotangent) to
// w2c_part[16 * block].
constexpr int kBwdThreads = 256;

template <int DEG, bool W2C, int SPAN>
__global__ __launch_bounds__(kBwdThreads) void preprocess_bwd_kernel(
    int64_t n, int K, const float* __restrict__ means, const float* __restrict__ scales,
    const float* __restrict__ quats, const float* __restrict__ opac, const float* __restrict__ sh,
    const float* __restrict__ w2c, float fx, float fy, const float* __restrict__ grec,
    float* __restrict__ g_means, float* __restrict__ g_scales, float* __restrict__ g_quats,
    float* __restrict__ g_opac, float* __restrict__ g_sh, float* __restrict__ w2c_part, int zeroed) {
  constexpr int NB = (DEG + 1) * (DEG + 1);
  constexpr int PER = SPAN / kBwdThreads;
  constexpr int NW = kBwdThreads / 64;
  __shared__ uint16_t reached_s[SPAN];
  __shared__ uint32_t wsum[NW];
  __shared__ float psum[NW][16];
  const int KC = 3 * K;
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int64_t g0 = (int64_t)blockIdx.x * SPAN;
  const bool aligned = (KC & 3) == 0 && (reinterpret_cast<uintptr_t>(sh) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(g_sh) & 15) == 0;
  const bool grec16 = (reinterpret_cast<uintptr_t>(grec) & 15) == 0;
  // 1. the span's records: thread t holds Gaussians g0 + t + kBwdThreads r
  bool hit[PER];
  uint32_t cnt = 0;
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int64_t i = g0 + t + kBwdThreads * r;
    hit[r] = false;
    if (i < n) {
      float grow[kRec];
      load_row<kRec>(grec + i * kRec, grec16, grow);
#pragma unroll
      for (int k = 0; k < 9; ++k) hit[r] = hit[r] || grow[k] != 0.0f;  // slots 9-11 hold nothing
    }
    cnt += hit[r] ? 1u : 0u;
  }
  // 2. list the reached ones (a block prefix sum of the counts), zero rows for the others
  uint32_t inc = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  if (lane == 63) wsum[wid] = inc;
  __syncthreads();
  uint32_t at = inc - cnt, total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    if (w < wid) at += wsum[w];
    total += wsum[w];
  }
#pragma unroll
  for (int r = 0; r < PER; ++r)
    if (hit[r]) reached_s[at++] = (uint16_t)(t + kBwdThreads * r);
  // unless the caller zeroed the arrays (zeroed: a compositing backward's clear list), the
  // span's gradient rows are zeroed whole, with coalesced 16-byte stores (a row per thread
  // took one partial cache line per lane and store); the reached rows are overwritten below,
  // after every zero store has completed
  if (!zeroed) {
    const int64_t g1 = g0 + SPAN < n ? g0 + SPAN : n;
    zero_block<kBwdThreads>(g_means, 3 * g0, 3 * g1, t);
    zero_block<kBwdThreads>(g_scales, 3 * g0, 3 * g1, t);
    zero_block<kBwdThreads>(g_quats, 4 * g0, 4 * g1, t);
    zero_block<kBwdThreads>(g_opac, g0, g1, t);
    zero_block<kBwdThreads>(g_sh, (int64_t)KC * g0, (int64_t)KC * g1, t);
    __builtin_amdgcn_s_waitcnt(0);  // the zero stores performed before any wave writes a row
  }
  __syncthreads();
  // 3. the reached Gaussians, one per thread
  float part[15];
#pragma unroll
  for (int k = 0; k < 15; ++k) part[k] = 0.0f;
  for (uint32_t j = t; j < total; j += kBwdThreads) {
    const int64_t i = g0 + reached_s[j];
    const GaussIn in = load_gauss(means, scales, quats, opac, i);
    float shv[3 * NB], grow[kRec];
    load_row<3 * NB>(sh + i * KC, aligned, shv);
    load_row<kRec>(grec + i * kRec, grec16, grow);
    float pg[15];  // this Gaussian's share (preprocess_bwd_gauss writes it whole)
    preprocess_bwd_gauss<DEG>(i, K, in, w2c, fx, fy, shv, grow, aligned, g_means, g_scales, g_quats, g_opac, g_sh,
                              W2C ? pg : nullptr);
    if (W2C) {
#pragma unroll
      for (int k = 0; k < 15; ++k) part[k] += pg[k];
    }
  }
  if (W2C) {
#pragma unroll
    for (int k = 0; k < 15; ++k) {
      const float v = wave_total(part[k]);
      if (lane == 0) psum[wid][k] = v;
    }
    __syncthreads();
    if (t < 15) {
      float v = psum[0][t];
#pragma unroll
      for (int w = 1; w < NW; ++w) v += psum[w][t];
      w2c_part[16 * (int64_t)blockIdx.x + t] = v;
    }
  }
}

// The VJP of composite_prep_kernel on its own (render_tiles' prologue, rasterizer.py:147-156):
// one thread per Gaussian, from its gradient record to the cotangents of means2D, cov2D
// (0 in [1,0], which render_tiles never reads), the opacity logit and the colour.
__global__ __launch_bounds__(256) void composite_prep_bwd_kernel(
    int64_t n, const float* __restrict__ cov2d, const float* __restrict__ opac, const float* __restrict__ grec,
    float* __restrict__ g_means2d, float* __restrict__ g_cov2d, float* __restrict__ g_opac,
    float* __restrict__ g_colors) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float4 c = reinterpret_cast<const float4*>(cov2d)[i];
  float grow[kRec];
  load_row<kRec>(grec + i * kRec, (reinterpret_cast<uintptr_t>(grec) & 15) == 0, grow);
  float g_m2x, g_m2y, G[2][2], g_logit;
  conic_vjp(grow, c.x, c.y, c.w, opac[i], g_m2x, g_m2y, G, g_logit);
  g_means2d[2 * i] = g_m2x;
  g_means2d[2 * i + 1] = g_m2y;
  reinterpret_cast<float4*>(g_cov2d)[i] = make_float4(G[0][0], G[0][1], G[1][0], G[1][1]);
  g_opac[i] = g_logit;
  g_colors[3 * i] = grow[6];
  g_colors[3 * i + 1] = grow[7];
  g_colors[3 * i + 2] = grow[8];
}

// The VJP of project_gaussians (projection.py:6-79) on its own: one thread per Gaussian,
// from the cotangents of means2D, cov2D (all four entries) and, with DEPTH, the depth z to
// those of the mean, log-scales and quaternion; with W2C each wave also writes its 64
// Gaussians' summed shares of dL/dW2C to w2c_part[16 * block] (the view-vector slots 12-14
// stay 0: project_gaussians computes no colour).
template <bool W2C, bool DEPTH>
__global__ __launch_bounds__(64) void project_bwd_kernel(
    int64_t n, const float* __restrict__ means, const float* __restrict__ scales, const float* __restrict__ quats,
    const float* __restrict__ w2c, float fx, float fy, const float* __restrict__ g_means2d,
    const float* __restrict__ g_cov2d, const float* __restrict__ g_depths, float* __restrict__ g_means,
    float* __restrict__ g_scales, float* __restrict__ g_quats, float* __restrict__ w2c_part) {
  const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  const int64_t ic = i < n ? i : n - 1;
  GaussIn in;
  in.mx = means[3 * ic];
  in.my = means[3 * ic + 1];
  in.mz = means[3 * ic + 2];
#pragma unroll
  for (int k = 0; k < 4; ++k) in.q[k] = quats[4 * ic + k];
#pragma unroll
  for (int k = 0; k < 3; ++k) in.ls[k] = scales[3 * ic + k];
  in.logit = 0.0f;
  float w[16];
  load_w2c(w2c, w);
  float part[15];
#pragma unroll
  for (int k = 0; k < 15; ++k) part[k] = 0.0f;
  if (i < n) {
    Proj p;
    project(w, in.mx, in.my, in.mz, in.q, in.ls, fx, fy, p);
    const float4 gc = reinterpret_cast<const float4*>(g_cov2d)[i];
    const float G[2][2] = {{gc.x, gc.y}, {gc.z, gc.w}};
    const float g_mcol[3] = {0.0f, 0.0f, 0.0f};
    project_vjp<DEPTH>(i, in, p, w, fx, fy, g_means2d[2 * i], g_means2d[2 * i + 1], G, DEPTH ? g_depths[i] : 0.0f,
                       g_mcol, g_means, g_scales, g_quats, W2C ? part : nullptr);
  }
  if (W2C) {
#pragma unroll
    for (int k = 0; k < 15; ++k) {
      const float t = wave_total(part[k]);
      if (threadIdx.x == 0) w2c_part[16 * (int64_t)blockIdx.x + k] = t;
    }
  }
}

// dL/dW2C from the waves' partial sums, in a fixed order (one workgroup): the shares through
// the mean and W_rot plus the camera centre's (centre = -R^T t, camera.py:15-21: with S
// the summed view-vector cotangent, dR[a][b] += t[a] S[b] and dt[a] += sum_b R[a][b] S[b]).
// Row 3 of W2C never enters the projection (projection.py:27 keeps three rows): zero.
__global__ __launch_bounds__(256) void w2c_finish_kernel(const float* __restrict__ part, int64_t nblk,
                                                         const float* __restrict__ w2c, float* __restrict__ g_w2c) {
  __shared__ float red[4][16];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  float acc[15];
#pragma unroll
  for (int k = 0; k < 15; ++k) acc[k] = 0.0f;
  for (int64_t b = tid; b < nblk; b += 256)
#pragma unroll
    for (int k = 0; k < 15; ++k) acc[k] += part[16 * b + k];
#pragma unroll
  for (int k = 0; k < 15; ++k) {
    const float t = wave_total(acc[k]);
    if (lane == 0) red[wid][k] = t;
  }
  __syncthreads();
  if (tid == 0) {
    float tot[15];
#pragma unroll
    for (int k = 0; k < 15; ++k) tot[k] = (red[0][k] + red[1][k]) + (red[2][k] + red[3][k]);
    for (int a = 0; a < 3; ++a) {
      float gt = tot[9 + a];
      for (int b = 0; b < 3; ++b) {
        g_w2c[4 * a + b] = tot[3 * a + b] + w2c[4 * a + 3] * tot[12 + b];
        gt += w2c[4 * a + b] * tot[12 + b];
      }
      g_w2c[4 * a + 3] = gt;
    }
    for (int b = 0; b < 4; ++b) g_w2c[12 + b] = 0.0f;
  }
}

// The training step's tail in one pass (trainer.py:137-159 with optax.adam of
// train.py:127-155): the preprocessing VJP as in preprocess_bwd_kernel, the
// densification statistics from the pre-update means, and the masked Adam update of
// all five arrays in place, so that no parameter gradient goes through HBM.  The
// per-element arithmetic is gs_adam_step's and the statistics are densify_kernel's, so
// the result equals the three-launch sequence bit for bit.
struct AdamConsts {
  float neg_lr[5];  // means, scales, quaternions, opacities, sh
  float b1, b2, omb1, omb2, bc1, bc2, eps;
};
struct MomentPtrs {
  float* mu[5];
  float* nu[5];
};

__device__ inline float adam_delta(const AdamConsts& A, int k, float g, float& m, float& v, bool on) {
  m = A.omb1 * g + A.b1 * m;
  v = A.omb2 * (g * g) + A.b2 * v;
  const float u = ((m / A.bc1) / (sqrtf(v / A.bc2) + A.eps)) * A.neg_lr[k];
  return on ? u : 0.0f;
}

template <int L>
__device__ inline void adam_row(const AdamConsts& A, int k, float* __restrict__ p, float* __restrict__ mu,
                                float* __restrict__ nu, const float* g, int64_t i, bool on) {
#pragma unroll
  for (int j = 0; j < L; ++j) {
    float m = mu[L * i + j], v = nu[L * i + j];
    const float d = adam_delta(A, k, g[j], m, v, on);
    p[L * i + j] = p[L * i + j] + d;
    mu[L * i + j] = m;
    nu[L * i + j] = v;
  }
}

template <int DEG>
__global__ __launch_bounds__(64) void preprocess_bwd_adam_kernel(
    int64_t n, int K, float* __restrict__ means, float* __restrict__ scales, float* __restrict__ quats,
    float* __restrict__ opac, float* __restrict__ sh, const float* __restrict__ w2c, float fx, float fy,
    const float* __restrict__ grec, MomentPtrs M, AdamConsts A, const uint8_t* __restrict__ active,
    const uint8_t* __restrict__ valid, const float* __restrict__ radii, float focal, float pixel_scale,
    float* __restrict__ grad_accum, int32_t* __restrict__ denom, float* __restrict__ max_radii) {
  constexpr int NB = (DEG + 1) * (DEG + 1);
  constexpr int LS = 49, LG = 13;
  __shared__ float shs[64 * LS];
  __shared__ float grs[64 * LG];
  const int lane = threadIdx.x;
  const int64_t g0 = (int64_t)blockIdx.x * 64;
  const int KC = 3 * K;
  const int64_t i = g0 + lane;
  const GaussIn in = load_gauss(means, scales, quats, opac, i < n ? i : n - 1);
  stage_rows<3 * NB>(sh, g0, n, (int64_t)KC, shs, LS, lane);
  stage_rows<kRec>(grec, g0, n, (int64_t)kRec, grs, LG, lane);
  __syncthreads();
  if (i < n) {
    float gm[3], gsc[3], gq[4], go[1];
    preprocess_bwd_one<DEG>(0, K, in, w2c, fx, fy, grs + lane * LG, shs + lane * LS, gm, gsc, gq, go);
    const bool on = active == nullptr || active[i] != 0;
    if (grad_accum != nullptr) {
      // trainer.py:143-159 from the means before the update
      const float zc = ((in.mx * w2c[8] + in.my * w2c[9]) + in.mz * w2c[10]) + w2c[11];
      const float z = jmax(zc, 0.01f);
      const float gn = sqrtf((gm[0] * gm[0] + gm[1] * gm[1]) + gm[2] * gm[2]);
      grad_accum[i] = grad_accum[i] + (gn * (z / focal)) * pixel_scale;
      const bool v = valid[i] != 0;
      denom[i] = denom[i] + ((v && on) ? 1 : 0);
      if (v) max_radii[i] = jmax(max_radii[i], radii[i]);
    }
    adam_row<3>(A, 0, means, M.mu[0], M.nu[0], gm, i, on);
    adam_row<3>(A, 1, scales, M.mu[1], M.nu[1], gsc, i, on);
    adam_row<4>(A, 2, quats, M.mu[2], M.nu[2], gq, i, on);
    adam_row<1>(A, 3, opac, M.mu[3], M.nu[3], go, i, on);
  }
  __syncthreads();
  // SH rows g0.. are contiguous: consecutive lanes update consecutive values (row of
  // element e as in preprocess_bwd_kernel)
  const float inv = 1.0f / (float)KC;
  const int64_t rows = n - g0 < 64 ? n - g0 : 64;
  const int total = (int)rows * KC;
  float* __restrict__ p = sh + g0 * KC;
  float* __restrict__ mu = M.mu[4] + g0 * KC;
  float* __restrict__ nu = M.nu[4] + g0 * KC;
  if ((KC & 3) == 0 && ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(mu) |
                         reinterpret_cast<uintptr_t>(nu)) & 15) == 0) {
    // 16-byte vectors, four in flight per lane (a row holds a whole number of vectors)
    const int nv = total >> 2;
    for (int v0 = lane; v0 < nv; v0 += 4 * 64) {
      float4 pp[4], mm[4], vv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int q = v0 + 64 * u;
        if (q < nv) {
          pp[u] = reinterpret_cast<const float4*>(p)[q];
          mm[u] = reinterpret_cast<const float4*>(mu)[q];
          vv[u] = reinterpret_cast<const float4*>(nu)[q];
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int q = v0 + 64 * u;
        if (q >= nv) continue;
        const int e = 4 * q;
        const int r = (int)(((float)e + 0.5f) * inv);
        const bool on = active == nullptr || active[g0 + r] != 0;
        const float* gr = shs + r * LS + (e - r * KC);
        pp[u].x = pp[u].x + adam_delta(A, 4, gr[0], mm[u].x, vv[u].x, on);
        pp[u].y = pp[u].y + adam_delta(A, 4, gr[1], mm[u].y, vv[u].y, on);
        pp[u].z = pp[u].z + adam_delta(A, 4, gr[2], mm[u].z, vv[u].z, on);
        pp[u].w = pp[u].w + adam_delta(A, 4, gr[3], mm[u].w, vv[u].w, on);
        reinterpret_cast<float4*>(p)[q] = pp[u];
        reinterpret_cast<float4*>(mu)[q] = mm[u];
        reinterpret_cast<float4*>(nu)[q] = vv[u];
      }
    }
  } else {
    for (int e = lane; e < total; e += 64) {
      const int r = (int)(((float)e + 0.5f) * inv);
      const bool on = active == nullptr || active[g0 + r] != 0;
      float m = mu[e], v = nu[e];
      const float d = adam_delta(A, 4, shs[r * LS + (e - r * KC)], m, v, on);
      p[e] = p[e] + d;
      mu[e] = m;
      nu[e] = v;
    }
  }
}

__global__ __launch_bounds__(256) void densify_kernel(int64_t n, const float* __restrict__ g_means,
                                                      const float* __restrict__ means,
                                                      const float* __restrict__ w2c, float focal,
                                                      float pixel_scale, const uint8_t* __restrict__ valid,
                                                      const uint8_t* __restrict__ active,
                                                      const float* __restrict__ radii,
                                                      float* __restrict__ grad_accum,
                                                      int32_t* __restrict__ denom,
                                                      float* __restrict__ max_radii) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // trainer.py:148-152; a zero cotangent (a Gaussian no pixel reached: most of them) adds +0,
  // which leaves the sum as it is, so its mean and sum are not read
  const float gx = g_means[3 * i], gy = g_means[3 * i + 1], gz = g_means[3 * i + 2];
  if (gx != 0.0f || gy != 0.0f || gz != 0.0f) {
    // trainer.py:145-147
    const float mx = means[3 * i], my = means[3 * i + 1], mz = means[3 * i + 2];
    const float zc = ((mx * w2c[8] + my * w2c[9]) + mz * w2c[10]) + w2c[11];
    const float z = jmax(zc, 0.01f);
    const float gn = sqrtf((gx * gx + gy * gy) + gz * gz);
    grad_accum[i] = grad_accum[i] + (gn * (z / focal)) * pixel_scale;
  }
  // trainer.py:153-159
  const bool v = valid[i] != 0;
  const bool act = (active == nullptr) || active[i] != 0;
  denom[i] = denom[i] + ((v && act) ? 1 : 0);
  if (v) max_radii[i] = jmax(max_radii[i], radii[i]);
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gs_preprocess_fwd(void* stream, int64_t n, int sh_k, int sh_degree, const float* means,
                                 const float* scales, const float* quats, const float* opacities,
                                 const float* sh_coeffs, const uint8_t* mask, const float* w2c,
                                 int width, int height, float fx, float fy, float cx, float cy,
                                 float* means2d, float* cov2d, float* radii, uint8_t* valid,
                                 float* depths, float* colors, float* records) {
  GS_REQUIRE(n >= 0, "gs_preprocess_fwd: n must be >= 0 (got %lld)", (long long)n);
  GS_REQUIRE(sh_degree >= 0 && sh_degree <= 3, "gs_preprocess_fwd: sh_degree must be in 0..3 (got %d)", sh_degree);
  GS_REQUIRE(sh_k >= (sh_degree + 1) * (sh_degree + 1),
             "gs_preprocess_fwd: sh_coeffs has %d coefficients, degree %d needs %d", sh_k, sh_degree,
             (sh_degree + 1) * (sh_degree + 1));
  GS_REQUIRE(width > 0 && height > 0, "gs_preprocess_fwd: bad image size %dx%d", width, height);
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && scales && quats && opacities && sh_coeffs && w2c && means2d && radii && valid && depths,
             "gs_preprocess_fwd: NULL array argument");
  GS_REQUIRE((cov2d && colors) || records, "gs_preprocess_fwd: cov2d and colors may be NULL only with records");
  (void)width;
  (void)height;
#define GS_PRE_FWD(D)                                                                                          \
  hipLaunchKernelGGL(preprocess_fwd_kernel<D>, dim3(div_up(n, 64)), dim3(64), 0, (hipStream_t)stream, n, sh_k,    \
                     means, scales, quats, opacities, sh_coeffs, mask, w2c, fx, fy, cx, cy, means2d, cov2d, radii, \
                     valid, depths, colors, records)
  switch (sh_degree) {
    case 0: GS_PRE_FWD(0); break;
    case 1: GS_PRE_FWD(1); break;
    case 2: GS_PRE_FWD(2); break;
    default: GS_PRE_FWD(3); break;
  }
#undef GS_PRE_FWD
  GS_LAUNCH_CHECK("preprocess_fwd_kernel");
  return GS_OK;
}

extern "C" int gs_composite_prep(void* stream, int64_t n, const float* means2d, const float* cov2d,
                                 const float* opacities, const float* colors, float* records) {
  GS_REQUIRE(n >= 0, "gs_composite_prep: n must be >= 0");
  if (n == 0) return GS_OK;
  GS_REQUIRE(means2d && cov2d && opacities && colors && records, "gs_composite_prep: NULL array argument");
  hipLaunchKernelGGL(composite_prep_kernel, dim3(div_up(n, 256)), dim3(256), 0, (hipStream_t)stream, n,
                     means2d, cov2d, opacities, colors, records);
  GS_LAUNCH_CHECK("composite_prep_kernel");
  return GS_OK;
}

namespace gs {
namespace {
// Gaussians per workgroup of preprocess_bwd_kernel: 1024 fills the GPU from about half a
// million Gaussians up (1M: 85 us against 90 with 256, 2M: 174 against 180); below, 256
// (200k: 26.5 us against 31).
inline int bwd_span(int64_t n) { return n < ((int64_t)1 << 19) ? 256 : 1024; }

int preprocess_bwd_launch(void* stream, int64_t n, int sh_k, int sh_degree, const float* means,
                          const float* scales, const float* quats, const float* opacities, const float* sh_coeffs,
                          const float* w2c, float fx, float fy, const float* grad_records, float* grad_means,
                          float* grad_scales, float* grad_quats, float* grad_opacities, float* grad_sh,
                          float* w2c_part, int zeroed, const char* who) {
  GS_REQUIRE(n >= 0, "%s: n must be >= 0", who);
  GS_REQUIRE(sh_degree >= 0 && sh_degree <= 3, "%s: sh_degree must be in 0..3 (got %d)", who, sh_degree);
  GS_REQUIRE(sh_k >= (sh_degree + 1) * (sh_degree + 1) && sh_k <= 16,
             "%s: sh_coeffs has %d coefficients, degree %d needs %d (max 16)", who, sh_k, sh_degree,
             (sh_degree + 1) * (sh_degree + 1));
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && scales && quats && opacities && sh_coeffs && w2c && grad_records && grad_means &&
                 grad_scales && grad_quats && grad_opacities && grad_sh,
             "%s: NULL array argument", who);
  const bool part = w2c_part != nullptr;
  const int span = bwd_span(n);
#define GS_PRE_BWD2(D, SP)                                                                                       \
  do {                                                                                                           \
    if (part)                                                                                                    \
      hipLaunchKernelGGL((preprocess_bwd_kernel<D, true, SP>), dim3(div_up(n, SP)), dim3(kBwdThreads), 0,        \
                         (hipStream_t)stream, n, sh_k, means, scales, quats, opacities, sh_coeffs, w2c, fx, fy,   \
                         grad_records, grad_means, grad_scales, grad_quats, grad_opacities, grad_sh, w2c_part,   \
                         zeroed);                                                                                \
    else                                                                                                         \
      hipLaunchKernelGGL((preprocess_bwd_kernel<D, false, SP>), dim3(div_up(n, SP)), dim3(kBwdThreads), 0,       \
                         (hipStream_t)stream, n, sh_k, means, scales, quats, opacities, sh_coeffs, w2c, fx, fy,   \
                         grad_records, grad_means, grad_scales, grad_quats, grad_opacities, grad_sh, nullptr,    \
                         zeroed);                                                                                \
  } while (0)
#define GS_PRE_BWD(D) \
  if (span == 1024) GS_PRE_BWD2(D, 1024); else GS_PRE_BWD2(D, 256)
  switch (sh_degree) {
    case 0: GS_PRE_BWD(0); break;
    case 1: GS_PRE_BWD(1); break;
    case 2: GS_PRE_BWD(2); break;
    default: GS_PRE_BWD(3); break;
  }
#undef GS_PRE_BWD
#undef GS_PRE_BWD2
  GS_LAUNCH_CHECK("preprocess_bwd_kernel");
  return GS_OK;
}
}  // namespace
}  // namespace gs

extern "C" int gs_preprocess_bwd(void* stream, int64_t n, int sh_k, int sh_degree, const float* means,
                                 const float* scales, const float* quats, const float* opacities,
                                 const float* sh_coeffs, const float* w2c, int width, int height,
                                 float fx, float fy, float cx, float cy, const float* grad_records,
                                 float* grad_means, float* grad_scales, float* grad_quats,
                                 float* grad_opacities, float* grad_sh, int zeroed) {
  (void)width;
  (void)height;
  (void)cx;
  (void)cy;
  return preprocess_bwd_launch(stream, n, sh_k, sh_degree, means, scales, quats, opacities, sh_coeffs, w2c, fx, fy,
                               grad_records, grad_means, grad_scales, grad_quats, grad_opacities, grad_sh, nullptr,
                               zeroed, "gs_preprocess_bwd");
}

extern "C" size_t gs_preprocess_bwd_w2c_workspace_size(int64_t n) {
  return n <= 0 ? 64 : (size_t)div_up(n, 64) * 16 * sizeof(float);
}

extern "C" int gs_preprocess_bwd_w2c(void* stream, int64_t n, int sh_k, int sh_degree, const float* means,
                                     const float* scales, const float* quats, const float* opacities,
                                     const float* sh_coeffs, const float* w2c, int width, int height, float fx,
                                     float fy, float cx, float cy, const float* grad_records, float* grad_means,
                                     float* grad_scales, float* grad_quats, float* grad_opacities, float* grad_sh,
                                     float* grad_w2c, void* workspace, size_t workspace_bytes, int zeroed) {
  (void)width;
  (void)height;
  (void)cx;
  (void)cy;
  GS_REQUIRE(grad_w2c != nullptr && w2c != nullptr, "gs_preprocess_bwd_w2c: NULL grad_w2c or w2c");
  GS_REQUIRE(workspace != nullptr && workspace_bytes >= gs_preprocess_bwd_w2c_workspace_size(n),
             "gs_preprocess_bwd_w2c: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
             gs_preprocess_bwd_w2c_workspace_size(n));
  const int rc = preprocess_bwd_launch(stream, n, sh_k, sh_degree, means, scales, quats, opacities, sh_coeffs, w2c,
                                       fx, fy, grad_records, grad_means, grad_scales, grad_quats, grad_opacities,
                                       grad_sh, (float*)workspace, zeroed, "gs_preprocess_bwd_w2c");
  if (rc != GS_OK) return rc;
  hipLaunchKernelGGL(w2c_finish_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, (const float*)workspace,
                     n > 0 ? div_up(n, bwd_span(n)) : (int64_t)0, w2c, grad_w2c);
  GS_LAUNCH_CHECK("w2c_finish_kernel");
  return GS_OK;
}

extern "C" int gs_composite_prep_bwd(void* stream, int64_t n, const float* cov2d, const float* opacities,
                                     const float* grad_records, float* grad_means2d, float* grad_cov2d,
                                     float* grad_opacities, float* grad_colors) {
  GS_REQUIRE(n >= 0, "gs_composite_prep_bwd: n must be >= 0");
  if (n == 0) return GS_OK;
  GS_REQUIRE(cov2d && opacities && grad_records && grad_means2d && grad_cov2d && grad_opacities && grad_colors,
             "gs_composite_prep_bwd: NULL array argument");
  hipLaunchKernelGGL(composite_prep_bwd_kernel, dim3(div_up(n, 256)), dim3(256), 0, (hipStream_t)stream, n, cov2d,
                     opacities, grad_records, grad_means2d, grad_cov2d, grad_opacities, grad_colors);
  GS_LAUNCH_CHECK("composite_prep_bwd_kernel");
  return GS_OK;
}

extern "C" int gs_project_bwd(void* stream, int64_t n, const float* means, const float* scales, const float* quats,
                              const float* w2c, float fx, float fy, const float* grad_means2d,
                              const float* grad_cov2d, const float* grad_depths, float* grad_means,
                              float* grad_scales, float* grad_quats, float* grad_w2c, void* workspace,
                              size_t workspace_bytes) {
  GS_REQUIRE(n >= 0, "gs_project_bwd: n must be >= 0");
  GS_REQUIRE(w2c != nullptr, "gs_project_bwd: NULL w2c");
  if (grad_w2c != nullptr)
    GS_REQUIRE(workspace != nullptr && workspace_bytes >= gs_preprocess_bwd_w2c_workspace_size(n),
               "gs_project_bwd: workspace of %zu bytes is smaller than the %zu required", workspace_bytes,
               gs_preprocess_bwd_w2c_workspace_size(n));
  hipStream_t s = (hipStream_t)stream;
  if (n > 0) {
    GS_REQUIRE(means && scales && quats && grad_means2d && grad_cov2d && grad_means && grad_scales && grad_quats,
               "gs_project_bwd: NULL array argument");
    float* part = (float*)workspace;
#define GS_PROJ_BWD(W, D)                                                                                        \
  hipLaunchKernelGGL((project_bwd_kernel<W, D>), dim3(div_up(n, 64)), dim3(64), 0, s, n, means, scales, quats, w2c, \
                     fx, fy, grad_means2d, grad_cov2d, grad_depths, grad_means, grad_scales, grad_quats, part)
    if (grad_w2c != nullptr) {
      if (grad_depths != nullptr) GS_PROJ_BWD(true, true);
      else GS_PROJ_BWD(true, false);
    } else {
      if (grad_depths != nullptr) GS_PROJ_BWD(false, true);
      else GS_PROJ_BWD(false, false);
    }
#undef GS_PROJ_BWD
    GS_LAUNCH_CHECK("project_bwd_kernel");
  }
  if (grad_w2c != nullptr) {
    hipLaunchKernelGGL(w2c_finish_kernel, dim3(1), dim3(256), 0, s, (const float*)workspace,
                       n > 0 ? div_up(n, 64) : (int64_t)0, w2c, grad_w2c);
    GS_LAUNCH_CHECK("w2c_finish_kernel");
  }
  return GS_OK;
}

namespace gs {
namespace {
// sh.py:25-74 on its own: one thread per row, the expansion without the renderer's +0.5
// and clip (eval_sh_channel, the reference's association order).
template <int DEG>
__global__ __launch_bounds__(256) void eval_sh_kernel(int64_t n, int K, const float* __restrict__ sh,
                                                      const float* __restrict__ dirs, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float d[3] = {dirs[3 * i], dirs[3 * i + 1], dirs[3 * i + 2]};
  const float* row = sh + i * 3 * K;
#pragma unroll
  for (int c = 0; c < 3; ++c) out[3 * i + c] = eval_sh_channel<DEG>(row, c, d);
}

// Its VJP: d colour_c / d s_kc = the signed factor E_k (exactly as the forward rounds it);
// d colour / d dir through the basis derivatives (JAX autodiff of sh.py:25-74).
template <int DEG>
__global__ __launch_bounds__(256) void eval_sh_bwd_kernel(int64_t n, int K, const float* __restrict__ sh,
                                                          const float* __restrict__ dirs,
                                                          const float* __restrict__ g_out, float* __restrict__ g_sh,
                                                          float* __restrict__ g_dirs) {
  constexpr int NB = (DEG + 1) * (DEG + 1);
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float d[3] = {dirs[3 * i], dirs[3 * i + 1], dirs[3 * i + 2]};
  const float g[3] = {g_out[3 * i], g_out[3 * i + 1], g_out[3 * i + 2]};
  float F[16];
  sh_factors<DEG>(d, F);
  float* dst = g_sh + i * 3 * K;
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const float e = (k == 1 || k == 3) ? -F[k] : F[k];
#pragma unroll
    for (int c = 0; c < 3; ++c) dst[3 * k + c] = e * g[c];
  }
  for (int q = 3 * NB; q < 3 * K; ++q) dst[q] = 0.0f;
  if (g_dirs == nullptr) return;
  float gd[3] = {0.0f, 0.0f, 0.0f};
  if (DEG > 0) {
    float B[16], dB[16][3];
    sh_basis_and_grad<DEG>(d, B, dB);
    const float* row = sh + i * 3 * K;
#pragma unroll
    for (int k = 1; k < NB; ++k) {
      const float sk = (row[3 * k] * g[0] + row[3 * k + 1] * g[1]) + row[3 * k + 2] * g[2];
#pragma unroll
      for (int j = 0; j < 3; ++j) gd[j] += sk * dB[k][j];
    }
  }
#pragma unroll
  for (int j = 0; j < 3; ++j) g_dirs[3 * i + j] = gd[j];
}
}  // namespace
}  // namespace gs

extern "C" int gs_eval_sh(void* stream, int64_t n, int sh_k, int sh_degree, const float* sh_coeffs,
                          const float* view_dirs, float* colors) {
  GS_REQUIRE(n >= 0, "gs_eval_sh: n must be >= 0");
  GS_REQUIRE(sh_degree >= 0 && sh_degree <= 3, "gs_eval_sh: sh_degree must be in 0..3 (got %d)", sh_degree);
  GS_REQUIRE(sh_k >= (sh_degree + 1) * (sh_degree + 1), "gs_eval_sh: sh_coeffs has %d coefficients, degree %d "
             "needs %d", sh_k, sh_degree, (sh_degree + 1) * (sh_degree + 1));
  if (n == 0) return GS_OK;
  GS_REQUIRE(sh_coeffs && view_dirs && colors, "gs_eval_sh: NULL array argument");
  hipStream_t s = (hipStream_t)stream;
  switch (sh_degree) {
    case 0: hipLaunchKernelGGL(eval_sh_kernel<0>, dim3(div_up(n, 256)), dim3(256), 0, s, n, sh_k, sh_coeffs, view_dirs, colors); break;
    case 1: hipLaunchKernelGGL(eval_sh_kernel<1>, dim3(div_up(n, 256)), dim3(256), 0, s, n, sh_k, sh_coeffs, view_dirs, colors); break;
    case 2: hipLaunchKernelGGL(eval_sh_kernel<2>, dim3(div_up(n, 256)), dim3(256), 0, s, n, sh_k, sh_coeffs, view_dirs, colors); break;
    default: hipLaunchKernelGGL(eval_sh_kernel<3>, dim3(div_up(n, 256)), dim3(256), 0, s, n, sh_k, sh_coeffs, view_dirs, colors); break;
  }
  GS_LAUNCH_CHECK("eval_sh_kernel");
  return GS_OK;
}

extern "C" int gs_eval_sh_bwd(void* stream, int64_t n, int sh_k, int sh_degree, const float* sh_coeffs,
                              const float* view_dirs, const float* grad_colors, float* grad_sh, float* grad_dirs) {
  GS_REQUIRE(n >= 0, "gs_eval_sh_bwd: n must be >= 0");
  GS_REQUIRE(sh_degree >= 0 && sh_degree <= 3, "gs_eval_sh_bwd: sh_degree must be in 0..3 (got %d)", sh_degree);
  GS_REQUIRE(sh_k >= (sh_degree + 1) * (sh_degree + 1), "gs_eval_sh_bwd: sh_coeffs has %d coefficients, degree "
             "%d needs %d", sh_k, sh_degree, (sh_degree + 1) * (sh_degree + 1));
  if (n == 0) return GS_OK;
  GS_REQUIRE(sh_coeffs && view_dirs && grad_colors && grad_sh, "gs_eval_sh_bwd: NULL array argument");
  hipStream_t s = (hipStream_t)stream;
#define GS_SH_BWD(D)                                                                                          \
  hipLaunchKernelGGL(eval_sh_bwd_kernel<D>, dim3(div_up(n, 256)), dim3(256), 0, s, n, sh_k, sh_coeffs, view_dirs, \
                     grad_colors, grad_sh, grad_dirs)
  switch (sh_degree) {
    case 0: GS_SH_BWD(0); break;
    case 1: GS_SH_BWD(1); break;
    case 2: GS_SH_BWD(2); break;
    default: GS_SH_BWD(3); break;
  }
#undef GS_SH_BWD
  GS_LAUNCH_CHECK("eval_sh_bwd_kernel");
  return GS_OK;
}

extern "C" int gs_densify_accumulate(void* stream, int64_t n, const float* grad_means, const float* means,
                                     const float* w2c, float focal, float pixel_scale,
                                     const uint8_t* valid, const uint8_t* active, const float* radii,
                                     float* grad_accum, int32_t* denom, float* max_radii) {
  GS_REQUIRE(n >= 0, "gs_densify_accumulate: n must be >= 0");
  if (n == 0) return GS_OK;
  GS_REQUIRE(grad_means && means && w2c && valid && radii && grad_accum && denom && max_radii,
             "gs_densify_accumulate: NULL array argument");
  hipLaunchKernelGGL(densify_kernel, dim3(div_up(n, 256)), dim3(256), 0, (hipStream_t)stream, n,
                     grad_means, means, w2c, focal, pixel_scale, valid, active, radii, grad_accum, denom,
                     max_radii);
  GS_LAUNCH_CHECK("densify_kernel");
  return GS_OK;
}

extern "C" int gs_preprocess_bwd_adam(void* stream, int64_t n, int sh_k, int sh_degree, float* means, float* scales,
                                      float* quats, float* opacities, float* sh_coeffs, const float* w2c, int width,
                                      int height, float fx, float fy, float cx, float cy, const float* grad_records,
                                      float* const* moments, const double* lrs, int step, double b1, double b2,
                                      double eps, const uint8_t* active, const uint8_t* valid, const float* radii,
                                      float focal, float pixel_scale, float* grad_accum, int32_t* denom,
                                      float* max_radii) {
  GS_REQUIRE(n >= 0, "gs_preprocess_bwd_adam: n must be >= 0");
  GS_REQUIRE(sh_degree >= 0 && sh_degree <= 3 && sh_k >= (sh_degree + 1) * (sh_degree + 1) && sh_k <= 16,
             "gs_preprocess_bwd_adam: sh_k %d / degree %d", sh_k, sh_degree);
  GS_REQUIRE(width > 0 && height > 0, "gs_preprocess_bwd_adam: bad image size %dx%d", width, height);
  GS_REQUIRE(step >= 1, "gs_preprocess_bwd_adam: step (count after this update) must be >= 1");
  GS_REQUIRE(moments && lrs, "gs_preprocess_bwd_adam: NULL moments / learning rates");
  if (n == 0) return GS_OK;
  GS_REQUIRE(means && scales && quats && opacities && sh_coeffs && w2c && grad_records,
             "gs_preprocess_bwd_adam: NULL array argument");
  GS_REQUIRE(grad_accum == nullptr || (denom && max_radii && valid && radii),
             "gs_preprocess_bwd_adam: statistics need denom, max_radii, valid and radii");
  MomentPtrs M;
  for (int k = 0; k < 5; ++k) {
    GS_REQUIRE(moments[k] && moments[5 + k], "gs_preprocess_bwd_adam: NULL moment array %d", k);
    M.mu[k] = moments[k];
    M.nu[k] = moments[5 + k];
  }
  // the same float32 constants as gs_adam_step
  AdamConsts A;
  for (int k = 0; k < 5; ++k) A.neg_lr[k] = (float)(-lrs[k]);
  A.b1 = (float)b1;
  A.b2 = (float)b2;
  A.omb1 = (float)(1.0 - b1);
  A.omb2 = (float)(1.0 - b2);
  A.bc1 = 1.0f - powf((float)b1, (float)step);
  A.bc2 = 1.0f - powf((float)b2, (float)step);
  A.eps = (float)eps;
  (void)cx;
  (void)cy;
#define GS_PRE_BWD_ADAM(D)                                                                                       \
  hipLaunchKernelGGL(preprocess_bwd_adam_kernel<D>, dim3(div_up(n, 64)), dim3(64), 0, (hipStream_t)stream, n,     \
                     sh_k, means, scales, quats, opacities, sh_coeffs, w2c, fx, fy, grad_records, M, A, active, valid, \
                     radii, focal, pixel_scale, grad_accum, denom, max_radii)
  switch (sh_degree) {
    case 0: GS_PRE_BWD_ADAM(0); break;
    case 1: GS_PRE_BWD_ADAM(1); break;
    case 2: GS_PRE_BWD_ADAM(2); break;
    default: GS_PRE_BWD_ADAM(3); break;
  }
#undef GS_PRE_BWD_ADAM
  GS_LAUNCH_CHECK("preprocess_bwd_adam_kernel");
  return GS_OK;
}
