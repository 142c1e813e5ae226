/*
 * Body of the CPU oracle, instantiated twice by gs_oracle.c: REAL=float (the
 * restatement the GPU path is compared with) and REAL=double (used only to check
 * the float restatement and its hand-derived backward by finite differences).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path links or calls this code.
 *
 * Each function restates the reference (ghif/jax-gs) operation by operation, in
 * the reference's association order, with no fused multiply-adds:
 *   preprocess_*        jax_gs/renderer/projection.py:6-79, jax_gs/core/gaussians.py:58-92,
 *                       jax_gs/core/camera.py:15-21, jax_gs/renderer/renderer.py:40-49,
 *                       jax_gs/renderer/sh.py:25-74
 *   tile_interactions_* jax_gs/renderer/rasterizer.py:12-116 (all 256*N slots, the
 *                       32-bit packed key, a stable sort, padding to 512)
 *   render_tiles_*      jax_gs/renderer/rasterizer.py:119-248 (searchsorted ranges, 8
 *                       chunks of 512 with the clamped dynamic_slice start, the
 *                       per-step gating, required_chunks, the empty-tile branch);
 *                       tpu_gather=1 selects the per-element clamped gather of
 *                       jax_gs/renderer/rasterizer_tpu.py:90-97 instead
 *   render_tiles_bwd_*  reverse-mode derivative of render_tiles as JAX autodiff
 *                       forms it: forward carries (T, C) kept per step, the cotangent
 *                       of T propagated backwards, gathers transposed to scatter-adds
 *   preprocess_bwd_*    reverse-mode derivative of preprocess_* (JAX conventions:
 *                       min/max/clip ties split 0.5/0.5, ceil has zero derivative)
 *   densify_*           jax_gs/training/trainer.py:143-159 (densification statistics)
 */

#define CAT2(a, b) a##_##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SFX)

static REAL FN(r_max)(REAL a, REAL b) { return (a != a || b != b) ? a + b : (a > b ? a : b); }
static REAL FN(r_min)(REAL a, REAL b) { return (a != a || b != b) ? a + b : (a < b ? a : b); }
/* share of the cotangent that jnp.maximum(a, b) / jnp.minimum(a, b) passes to a */
static REAL FN(d_max)(REAL a, REAL b) { return a > b ? (REAL)1 : (a == b ? (REAL)0.5 : (REAL)0); }
static REAL FN(d_min)(REAL a, REAL b) { return a < b ? (REAL)1 : (a == b ? (REAL)0.5 : (REAL)0); }

static const REAL FN(C0) = (REAL)0.28209479177387814;
static const REAL FN(C1) = (REAL)0.4886025119029199;
static const REAL FN(C2)[5] = {(REAL)1.0925484305920792, (REAL)-1.0925484305920792, (REAL)0.31539156525252005,
                               (REAL)-1.0925484305920792, (REAL)0.5462742152960396};
static const REAL FN(C3)[7] = {(REAL)-0.5900435899266435, (REAL)2.890611442640554, (REAL)-0.4570457994644658,
                               (REAL)0.3731763325901154, (REAL)-0.4570457994644658, (REAL)1.445305721320277,
                               (REAL)-0.5900435899266435};

typedef struct {
  REAL x, y, z;
  REAL q[4], qn[4], qnorm;
  REAL R[3][3], s[3], Mm[3][3], Sig[3][3];
  REAL zs, iz, iz2, J[2][3], M2[2][3], T1[2][3];
  REAL cov[2][2];
} FN(proj_t);

static void FN(project)(const REAL* w, const REAL* m, const REAL* q, const REAL* ls, REAL fx, REAL fy,
                        FN(proj_t) * p) {
  int i, j;
  /* projection.py:26-29 */
  p->x = ((m[0] * w[0] + m[1] * w[1]) + m[2] * w[2]) + w[3];
  p->y = ((m[0] * w[4] + m[1] * w[5]) + m[2] * w[6]) + w[7];
  p->z = ((m[0] * w[8] + m[1] * w[9]) + m[2] * w[10]) + w[11];
  /* gaussians.py:70-91 */
  for (i = 0; i < 4; ++i) p->q[i] = q[i];
  p->qnorm = SQRT(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
  for (i = 0; i < 4; ++i) p->qn[i] = q[i] / p->qnorm;
  {
    const REAL r = p->qn[0], x = p->qn[1], y = p->qn[2], z = p->qn[3];
    const REAL one = 1, two = 2;
    p->R[0][0] = (one - two * (y * y)) - two * (z * z);
    p->R[0][1] = (two * x) * y - (two * r) * z;
    p->R[0][2] = (two * x) * z + (two * r) * y;
    p->R[1][0] = (two * x) * y + (two * r) * z;
    p->R[1][1] = (one - two * (x * x)) - two * (z * z);
    p->R[1][2] = (two * y) * z - (two * r) * x;
    p->R[2][0] = (two * x) * z - (two * r) * y;
    p->R[2][1] = (two * y) * z + (two * r) * x;
    p->R[2][2] = (one - two * (x * x)) - two * (y * y);
  }
  for (j = 0; j < 3; ++j) p->s[j] = EXP(ls[j]);
  for (i = 0; i < 3; ++i)
    for (j = 0; j < 3; ++j) p->Mm[i][j] = p->R[i][j] * p->s[j];
  for (i = 0; i < 3; ++i)
    for (j = 0; j < 3; ++j)
      p->Sig[i][j] = (p->Mm[i][0] * p->Mm[j][0] + p->Mm[i][1] * p->Mm[j][1]) + p->Mm[i][2] * p->Mm[j][2];
  /* projection.py:43-62 */
  p->zs = FN(r_max)(p->z, (REAL)0.01);
  p->iz = (REAL)1 / p->zs;
  p->iz2 = p->iz * p->iz;
  p->J[0][0] = fx * p->iz;
  p->J[0][1] = 0;
  p->J[0][2] = ((-fx) * p->x) * p->iz2;
  p->J[1][0] = 0;
  p->J[1][1] = fy * p->iz;
  p->J[1][2] = ((-fy) * p->y) * p->iz2;
  for (i = 0; i < 2; ++i)
    for (j = 0; j < 3; ++j)
      p->M2[i][j] = (p->J[i][0] * w[0 * 4 + j] + p->J[i][1] * w[1 * 4 + j]) + p->J[i][2] * w[2 * 4 + j];
  for (i = 0; i < 2; ++i)
    for (j = 0; j < 3; ++j)
      p->T1[i][j] = (p->M2[i][0] * p->Sig[0][j] + p->M2[i][1] * p->Sig[1][j]) + p->M2[i][2] * p->Sig[2][j];
  for (i = 0; i < 2; ++i)
    for (j = 0; j < 2; ++j)
      p->cov[i][j] = (p->T1[i][0] * p->M2[j][0] + p->T1[i][1] * p->M2[j][1]) + p->T1[i][2] * p->M2[j][2];
  p->cov[0][0] = p->cov[0][0] + (REAL)0.3;
  p->cov[0][1] = p->cov[0][1] + (REAL)0;
  p->cov[1][0] = p->cov[1][0] + (REAL)0;
  p->cov[1][1] = p->cov[1][1] + (REAL)0.3;
}

static void FN(viewdir)(const REAL* w, const REAL* m, REAL* v, REAL* nrm, REAL* d) {
  int i;
  REAL cen[3];
  for (i = 0; i < 3; ++i) cen[i] = ((-w[0 * 4 + i]) * w[3] + (-w[1 * 4 + i]) * w[7]) + (-w[2 * 4 + i]) * w[11];
  for (i = 0; i < 3; ++i) v[i] = m[i] - cen[i];
  *nrm = SQRT((v[0] * v[0] + v[1] * v[1]) + v[2] * v[2]);
  for (i = 0; i < 3; ++i) d[i] = v[i] / *nrm;
}

/* sh.py:25-72, one channel c of Gaussian coefficients sh[K][3] */
static REAL FN(eval_sh)(int deg, const REAL* sh, int c, const REAL* d) {
  const REAL* C2 = FN(C2);
  const REAL* C3 = FN(C3);
  REAL res = FN(C0) * sh[0 * 3 + c];
  if (deg > 0) {
    const REAL x = d[0], y = d[1], z = d[2];
    res = ((res - (FN(C1) * y) * sh[1 * 3 + c]) + (FN(C1) * z) * sh[2 * 3 + c]) - (FN(C1) * x) * sh[3 * 3 + c];
    if (deg > 1) {
      const REAL xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
      res = ((((res + (C2[0] * xy) * sh[4 * 3 + c]) + (C2[1] * yz) * sh[5 * 3 + c]) +
              (C2[2] * (((REAL)2 * zz - xx) - yy)) * sh[6 * 3 + c]) +
             (C2[3] * xz) * sh[7 * 3 + c]) +
            (C2[4] * (xx - yy)) * sh[8 * 3 + c];
      if (deg > 2) {
        res = ((((((res + ((C3[0] * y) * ((REAL)3 * xx - yy)) * sh[9 * 3 + c]) + ((C3[1] * xy) * z) * sh[10 * 3 + c]) +
                  ((C3[2] * y) * (((REAL)4 * zz - xx) - yy)) * sh[11 * 3 + c]) +
                 ((C3[3] * z) * (((REAL)2 * zz - (REAL)3 * xx) - (REAL)3 * yy)) * sh[12 * 3 + c]) +
                ((C3[4] * x) * (((REAL)4 * zz - xx) - yy)) * sh[13 * 3 + c]) +
               ((C3[5] * z) * (xx - yy)) * sh[14 * 3 + c]) +
              ((C3[6] * x) * (xx - (REAL)3 * yy)) * sh[15 * 3 + c];
      }
    }
  }
  return res;
}

int FN(gso_preprocess)(int64_t n, int K, int deg, const REAL* means, const REAL* scales, const REAL* quats,
                       const REAL* opac, const REAL* sh, const uint8_t* mask, const REAL* w2c, int W, int H,
                       REAL fx, REAL fy, REAL cx, REAL cy, REAL* means2d, REAL* cov2d, REAL* radii,
                       uint8_t* valid, REAL* depths, REAL* colors) {
  int64_t i;
  (void)opac;
  (void)W;
  (void)H;
#pragma omp parallel for schedule(static)
  for (i = 0; i < n; ++i) {
    FN(proj_t) p;
    REAL v[3], nrm, d[3];
    int c;
    FN(project)(w2c, means + 3 * i, quats + 4 * i, scales + 3 * i, fx, fy, &p);
    valid[i] = (p.z > (REAL)0.01) && (mask == NULL || mask[i] != 0);
    means2d[2 * i] = (fx * p.x) / p.z + cx;
    means2d[2 * i + 1] = (fy * p.y) / p.z + cy;
    cov2d[4 * i + 0] = p.cov[0][0];
    cov2d[4 * i + 1] = p.cov[0][1];
    cov2d[4 * i + 2] = p.cov[1][0];
    cov2d[4 * i + 3] = p.cov[1][1];
    {
      const REAL det = p.cov[0][0] * p.cov[1][1] - p.cov[0][1] * p.cov[0][1];
      const REAL mid = (p.cov[0][0] + p.cov[1][1]) / (REAL)2;
      const REAL term = SQRT(FN(r_max)(mid * mid - det, (REAL)0));
      radii[i] = CEIL((REAL)3 * SQRT(mid + term));
    }
    depths[i] = p.z;
    FN(viewdir)(w2c, means + 3 * i, v, &nrm, d);
    for (c = 0; c < 3; ++c) {
      const REAL res = FN(eval_sh)(deg, sh + (int64_t)i * K * 3, c, d) + (REAL)0.5;
      colors[3 * i + c] = FN(r_min)(FN(r_max)((REAL)0, res), (REAL)1);
    }
  }
  return 0;
}

/* rasterizer.py:12-116.  sorted_tiles / sorted_gids have length L = max(256n, 512). */
int FN(gso_tile_interactions)(int64_t n, const REAL* means2d, const REAL* radii, const uint8_t* valid,
                              const REAL* depths, int W, int H, int32_t* sorted_tiles, int32_t* sorted_gids,
                              int64_t* n_interactions) {
  const int TX = (W + 15) / 16, TY = (H + 15) / 16, T = TX * TY;
  const int64_t total = n * 256;
  const int64_t L = total > 512 ? total : 512;
  uint32_t *key = NULL, *val = NULL, *k2 = NULL, *v2 = NULL;
  int64_t i, cnt = 0;
  int pass;
  gso_hint_huge(sorted_tiles, sizeof(int32_t) * (size_t)L);
  gso_hint_huge(sorted_gids, sizeof(int32_t) * (size_t)L);
  if (total > 0) {
    key = (uint32_t*)gso_big_alloc(sizeof(uint32_t) * total);
    val = (uint32_t*)gso_big_alloc(sizeof(uint32_t) * total);
    k2 = (uint32_t*)gso_big_alloc(sizeof(uint32_t) * total);
    v2 = (uint32_t*)gso_big_alloc(sizeof(uint32_t) * total);
    if (!key || !val || !k2 || !v2) {
      free(key); free(val); free(k2); free(v2);
      return -1;
    }
  }
#pragma omp parallel for schedule(static) reduction(+ : cnt)
  for (i = 0; i < n; ++i) {
    const REAL mx = means2d[2 * i], my = means2d[2 * i + 1], r = radii[i];
    const REAL minx = FN(r_min)(FN(r_max)(mx - r, (REAL)0), (REAL)(W - 1));
    const REAL maxx = FN(r_min)(FN(r_max)(mx + r, (REAL)0), (REAL)(W - 1));
    const REAL miny = FN(r_min)(FN(r_max)(my - r, (REAL)0), (REAL)(H - 1));
    const REAL maxy = FN(r_min)(FN(r_max)(my + r, (REAL)0), (REAL)(H - 1));
    /* (x // 16).astype(int32): floor division, then conversion (NaN -> 0 as XLA does) */
    const REAL fminx = FLOOR(minx / (REAL)16), fmaxx = FLOOR(maxx / (REAL)16);
    const REAL fminy = FLOOR(miny / (REAL)16), fmaxy = FLOOR(maxy / (REAL)16);
    const int tminx = fminx == fminx ? (int)fminx : 0, tmaxx = fmaxx == fmaxx ? (int)fmaxx : 0;
    const int tminy = fminy == fminy ? (int)fminy : 0, tmaxy = fmaxy == fmaxy ? (int)fmaxy : 0;
    const int on = (mx + r > 0) && (mx - r < (REAL)W) && (my + r > 0) && (my - r < (REAL)H);
    const int v = valid[i] && on && (tmaxx >= tminx) && (tmaxy >= tminy);
    float zf = (float)depths[i];
    int32_t zb, dq;
    int oy, ox;
    memcpy(&zb, &zf, 4);
    dq = zb >> (31 - 13); /* arithmetic shift */
    for (oy = 0; oy < 16; ++oy)
      for (ox = 0; ox < 16; ++ox) {
        const int ax = tminx + ox, ay = tminy + oy;
        const int in_range = (ax <= tmaxx) && (ay <= tmaxy) && v;
        const int32_t tile = in_range ? ay * TX + ax : T; /* sentinel for no interaction */
        const int32_t k = (int32_t)(((uint32_t)tile << 13) | (uint32_t)dq);
        const int64_t slot = i * 256 + oy * 16 + ox;
        key[slot] = (uint32_t)k ^ 0x80000000u; /* signed order as unsigned */
        val[slot] = (uint32_t)i;
        cnt += in_range;
      }
  }
  /* stable LSD radix sort, 4 x 8 bits.  Each thread owns a contiguous block of the
   * array; per-thread digit counts are turned into destinations in (digit, thread)
   * order, so equal digits keep their input order across blocks (stability). */
  if (total > 0) {
    const int nt_max = omp_get_max_threads();
    int64_t* th = (int64_t*)calloc((size_t)nt_max * 256, sizeof(int64_t));
    if (!th) {
      free(key); free(val); free(k2); free(v2);
      return -1;
    }
    for (pass = 0; pass < 4; ++pass) {
      const int sh = pass * 8;
      uint32_t* t;
#pragma omp parallel num_threads(nt_max)
      {
        const int tid = omp_get_thread_num(), nth = omp_get_num_threads();
        const int64_t lo = total * tid / nth, hi = total * (tid + 1) / nth;
        int64_t* h = th + (size_t)tid * 256;
        int64_t j;
        memset(h, 0, sizeof(int64_t) * 256);
        for (j = lo; j < hi; ++j) h[(key[j] >> sh) & 255]++;
#pragma omp barrier
#pragma omp single
        {
          int64_t run = 0, c;
          int dg, tt;
          for (dg = 0; dg < 256; ++dg)
            for (tt = 0; tt < nth; ++tt) {
              c = th[(size_t)tt * 256 + dg];
              th[(size_t)tt * 256 + dg] = run;
              run += c;
            }
        }
        for (j = lo; j < hi; ++j) {
          const int64_t dst = h[(key[j] >> sh) & 255]++;
          k2[dst] = key[j];
          v2[dst] = val[j];
        }
      }
      t = key; key = k2; k2 = t;
      t = val; val = v2; v2 = t;
    }
    free(th);
  }
#pragma omp parallel for schedule(static)
  for (i = 0; i < L; ++i) {
    if (i < total) {
      const int32_t k = (int32_t)(key[i] ^ 0x80000000u);
      sorted_tiles[i] = k >> 13;
      sorted_gids[i] = (int32_t)val[i];
    } else {
      sorted_tiles[i] = T;
      sorted_gids[i] = 0;
    }
  }
  *n_interactions = cnt;
  free(key); free(val); free(k2); free(v2);
  return 0;
}

/* jnp.searchsorted(a, v, side='left') */
static int64_t FN(lower_bound)(const int32_t* a, int64_t len, int64_t v) {
  int64_t lo = 0, hi = len;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if ((int64_t)a[mid] < v)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

/* Per-tile setup shared by the forward and backward restatements. */
typedef struct {
  int64_t start;
  int count;          /* min(end - start, 4096) */
  int required;       /* required_chunks */
} FN(tile_t);

static void FN(tile_setup)(const int32_t* sorted_tiles, int64_t L, int t, FN(tile_t) * ts) {
  const int64_t s = FN(lower_bound)(sorted_tiles, L, t);
  const int64_t e = FN(lower_bound)(sorted_tiles, L, (int64_t)t + 1);
  int64_t c = e - s;
  if (c > 4096) c = 4096;
  ts->start = s;
  ts->count = (int)c;
  ts->required = (int)((c + 511) / 512);
  if (ts->required < 1) ts->required = 1;
}

/* Gaussian id used at step i of chunk ch (rasterizer.py:188-190, or the TPU path's
 * per-element clamp rasterizer_tpu.py:93-97). */
static int64_t FN(entry_index)(const FN(tile_t) * ts, int ch, int i, int64_t L, int tpu_gather) {
  const int64_t chunk_start = ts->start + (int64_t)ch * 512;
  if (tpu_gather) {
    int64_t idx = chunk_start + i;
    if (idx > L - 1) idx = L - 1;
    if (idx < 0) idx = 0;
    return idx;
  } else {
    int64_t hi = L - 512;
    int64_t gs;
    if (hi < 0) hi = 0;
    gs = chunk_start < 0 ? 0 : (chunk_start > hi ? hi : chunk_start);
    return gs + i;
  }
}

typedef struct {
  REAL mx, my, ic00, ic01_2, ic11, op, col[3];
} FN(prim_t);

static void FN(prim_of)(const REAL* means2d, const REAL* cov2d, const REAL* opac, const REAL* colors,
                        int64_t g, FN(prim_t) * pr) {
  /* rasterizer.py:147-156 and 197-200 */
  const REAL c00 = cov2d[4 * g], c01 = cov2d[4 * g + 1], c11 = cov2d[4 * g + 3];
  const REAL det = FN(r_max)(c00 * c11 - c01 * c01, (REAL)1e-6);
  pr->mx = means2d[2 * g];
  pr->my = means2d[2 * g + 1];
  pr->ic00 = c11 / det;
  pr->ic01_2 = (REAL)2 * ((-c01) / det);
  pr->ic11 = c00 / det;
  pr->op = SIGMOID(opac[g]);
  pr->col[0] = colors[3 * g];
  pr->col[1] = colors[3 * g + 1];
  pr->col[2] = colors[3 * g + 2];
}

static REAL FN(power)(REAL dx, REAL dy, const FN(prim_t) * pr, int tpu_form) {
  if (tpu_form) /* rasterizer_tpu.py:78 */
    return (REAL)-0.5 * ((dx * dx * pr->ic00 + (REAL)2 * dx * dy * (pr->ic01_2 / (REAL)2)) + dy * dy * pr->ic11);
  return (REAL)-0.5 * (((dx * dx) * pr->ic00 + (dx * dy) * pr->ic01_2) + (dy * dy) * pr->ic11);
}

/* rasterizer.py:119-248 (tpu_gather=0) / rasterizer_tpu.py:13-135 (tpu_gather=1).
 * image[H,W,3]; final_T[H,W] and n_contrib[H,W] may be NULL. */
int FN(gso_render_tiles)(int64_t n, const REAL* means2d, const REAL* cov2d, const REAL* opac, const REAL* colors,
                         const int32_t* sorted_tiles, const int32_t* sorted_gids, int64_t L, int W, int H,
                         const REAL* bg, int tpu_gather, REAL* image, REAL* final_T, int32_t* n_contrib) {
  const int TX = (W + 15) / 16, TY = (H + 15) / 16, T = TX * TY;
  int t;
  (void)n;
#pragma omp parallel for schedule(dynamic, 1)
  for (t = 0; t < T; ++t) {
    const int tx = t % TX, ty = t / TX;
    FN(tile_t) ts;
    int pi;
    FN(tile_setup)(sorted_tiles, L, t, &ts);
    for (pi = 0; pi < 256; ++pi) {
      const int lx = pi % 16, ly = pi / 16;
      const int X = tx * 16 + lx, Y = ty * 16 + ly;
      const REAL px = (REAL)(tx * 16) + ((REAL)lx + (REAL)0.5);
      const REAL py = (REAL)(ty * 16) + ((REAL)ly + (REAL)0.5);
      REAL C[3] = {0, 0, 0}, Tr = 1;
      int last = 0, ch, i;
      if (X >= W || Y >= H) continue;
      if (ts.count > 0) {
        for (ch = 0; ch < 8; ++ch) {
          if (ch >= (tpu_gather ? 8 : ts.required)) break;
          for (i = 0; i < 512; ++i) {
            const int local = ch * 512 + i;
            const int64_t gidx = FN(entry_index)(&ts, ch, i, L, tpu_gather);
            const int64_t g = sorted_gids[gidx];
            FN(prim_t) pr;
            REAL dx, dy, pw, alpha;
            int active;
            if (!(local < ts.count)) continue;
            active = Tr > (REAL)1e-4;
            if (!active) continue;
            FN(prim_of)(means2d, cov2d, opac, colors, g, &pr);
            dx = px - pr.mx;
            dy = py - pr.my;
            pw = FN(power)(dx, dy, &pr, tpu_gather);
            alpha = EXP(pw) * pr.op;
            alpha = pw > (REAL)-10 ? FN(r_min)((REAL)0.99, alpha) : (REAL)0;
            C[0] = C[0] + (alpha * Tr) * pr.col[0];
            C[1] = C[1] + (alpha * Tr) * pr.col[1];
            C[2] = C[2] + (alpha * Tr) * pr.col[2];
            Tr = Tr * ((REAL)1 - alpha);
            last = local + 1;
          }
        }
        image[3 * ((int64_t)Y * W + X) + 0] = C[0] + Tr * bg[0];
        image[3 * ((int64_t)Y * W + X) + 1] = C[1] + Tr * bg[1];
        image[3 * ((int64_t)Y * W + X) + 2] = C[2] + Tr * bg[2];
      } else {
        image[3 * ((int64_t)Y * W + X) + 0] = bg[0];
        image[3 * ((int64_t)Y * W + X) + 1] = bg[1];
        image[3 * ((int64_t)Y * W + X) + 2] = bg[2];
      }
      if (final_T) final_T[(int64_t)Y * W + X] = Tr;
      if (n_contrib) n_contrib[(int64_t)Y * W + X] = last;
    }
  }
  return 0;
}

/* Reverse-mode derivative of gso_render_tiles.  Outputs are overwritten:
 * g_means2d[n,2], g_cov2d[n,4] (the [1,0] entry stays 0), g_opac[n] (w.r.t. the
 * logit), g_colors[n,3], g_bg[3]. */
int FN(gso_render_tiles_bwd)(int64_t n, const REAL* means2d, const REAL* cov2d, const REAL* opac,
                             const REAL* colors, const int32_t* sorted_tiles, const int32_t* sorted_gids, int64_t L,
                             int W, int H, const REAL* bg, int tpu_gather, const REAL* g_image, REAL* g_means2d,
                             REAL* g_cov2d, REAL* g_opac, REAL* g_colors, REAL* g_bg) {
  const int TX = (W + 15) / 16, TY = (H + 15) / 16, T = TX * TY;
  /* Per-thread cotangent accumulators (the reference's gather transposes are
   * scatter-adds, whose order XLA leaves unspecified): 9 values per Gaussian, laid out
   * [ic00, ic01_2, ic11 | sigmoid | means2d x, y | colour r, g, b] blocks of n each,
   * summed in thread order after the tiles. */
  const int nt_max = omp_get_max_threads();
  const size_t nn = (size_t)(n > 0 ? n : 1);
  REAL* acc = (REAL*)calloc(nn * 9 * (size_t)nt_max, sizeof(REAL));
  REAL* bgacc = (REAL*)calloc((size_t)nt_max * 3, sizeof(REAL));
  int64_t g;
  int fail = 0;
  if (!acc || !bgacc) {
    free(acc); free(bgacc);
    return -1;
  }
#pragma omp parallel num_threads(nt_max) reduction(| : fail)
  {
    const int tid = omp_get_thread_num();
    REAL* a = acc + nn * 9 * (size_t)tid;
    REAL* g_ic = a;             /* [n][3] */
    REAL* g_sig = a + 3 * nn;   /* [n] */
    REAL* g_m2 = a + 4 * nn;    /* [n][2] */
    REAL* g_col = a + 6 * nn;   /* [n][3] */
    REAL* g_b = bgacc + 3 * tid;
    REAL* Tk = (REAL*)malloc(sizeof(REAL) * 4097);
    int64_t* gk = (int64_t*)malloc(sizeof(int64_t) * 4096);
    int t;
    if (!Tk || !gk) fail = 1;
#pragma omp for schedule(dynamic, 1)
    for (t = 0; t < T; ++t) {
      const int tx = t % TX, ty = t / TX;
      FN(tile_t) ts;
      int pi;
      if (!Tk || !gk) continue;
      FN(tile_setup)(sorted_tiles, L, t, &ts);
      for (pi = 0; pi < 256; ++pi) {
        const int lx = pi % 16, ly = pi / 16;
        const int X = tx * 16 + lx, Y = ty * 16 + ly;
        const REAL px = (REAL)(tx * 16) + ((REAL)lx + (REAL)0.5);
        const REAL py = (REAL)(ty * 16) + ((REAL)ly + (REAL)0.5);
        const REAL* gp;
        REAL ctC[3], ctT;
        int k, nk = 0, ch, i;
        if (X >= W || Y >= H) continue;
        gp = g_image + 3 * ((int64_t)Y * W + X);
        if (ts.count == 0) { /* empty tile: image = background */
          g_b[0] += gp[0]; g_b[1] += gp[1]; g_b[2] += gp[2];
          continue;
        }
        /* forward replay, keeping T before every step */
        Tk[0] = 1;
        for (ch = 0; ch < 8; ++ch) {
          if (ch >= (tpu_gather ? 8 : ts.required)) break;
          for (i = 0; i < 512; ++i) {
            const int local = ch * 512 + i;
            if (!(local < ts.count)) continue;
            gk[nk] = sorted_gids[FN(entry_index)(&ts, ch, i, L, tpu_gather)];
            {
              FN(prim_t) pr;
              REAL dx, dy, pw, alpha = 0;
              FN(prim_of)(means2d, cov2d, opac, colors, gk[nk], &pr);
              if (Tk[nk] > (REAL)1e-4) {
                dx = px - pr.mx; dy = py - pr.my;
                pw = FN(power)(dx, dy, &pr, tpu_gather);
                alpha = pw > (REAL)-10 ? FN(r_min)((REAL)0.99, EXP(pw) * pr.op) : (REAL)0;
              }
              Tk[nk + 1] = Tk[nk] * ((REAL)1 - alpha);
            }
            ++nk;
          }
        }
        /* out = C_n + T_n * bg */
        ctC[0] = gp[0]; ctC[1] = gp[1]; ctC[2] = gp[2];
        ctT = (gp[0] * bg[0] + gp[1] * bg[1]) + gp[2] * bg[2];
        g_b[0] += Tk[nk] * gp[0]; g_b[1] += Tk[nk] * gp[1]; g_b[2] += Tk[nk] * gp[2];
        for (k = nk - 1; k >= 0; --k) {
          FN(prim_t) pr;
          REAL dx, dy, pw, e, araw, alpha, ct_alpha, ct_araw, ct_pw, cdot;
          const REAL Tb = Tk[k];
          const int64_t gg = gk[k];
          if (!(Tb > (REAL)1e-4)) continue; /* inactive: C and T pass through */
          FN(prim_of)(means2d, cov2d, opac, colors, gg, &pr);
          dx = px - pr.mx; dy = py - pr.my;
          pw = FN(power)(dx, dy, &pr, tpu_gather);
          if (!(pw > (REAL)-10)) continue; /* alpha = 0: pass through, no cotangent */
          e = EXP(pw);
          araw = e * pr.op;
          alpha = FN(r_min)((REAL)0.99, araw);
          /* C' = C + (alpha T) col ; T' = T (1 - alpha) */
          cdot = (pr.col[0] * ctC[0] + pr.col[1] * ctC[1]) + pr.col[2] * ctC[2];
          ct_alpha = Tb * cdot - Tb * ctT;
          g_col[3 * gg + 0] += (alpha * Tb) * ctC[0];
          g_col[3 * gg + 1] += (alpha * Tb) * ctC[1];
          g_col[3 * gg + 2] += (alpha * Tb) * ctC[2];
          ctT = alpha * cdot + ((REAL)1 - alpha) * ctT;
          ct_araw = ct_alpha * FN(d_min)(araw, (REAL)0.99);
          g_sig[gg] += ct_araw * e;
          ct_pw = ct_araw * araw;
          {
            const REAL h = (REAL)-0.5 * ct_pw;
            const REAL ctdx = h * ((REAL)2 * dx * pr.ic00 + dy * pr.ic01_2);
            const REAL ctdy = h * (dx * pr.ic01_2 + (REAL)2 * dy * pr.ic11);
            g_ic[3 * gg + 0] += h * (dx * dx);
            g_ic[3 * gg + 1] += h * (dx * dy);
            g_ic[3 * gg + 2] += h * (dy * dy);
            g_m2[2 * gg] -= ctdx;
            g_m2[2 * gg + 1] -= ctdy;
          }
        }
      }
    }
    free(Tk);
    free(gk);
  }
  if (fail) {
    free(acc); free(bgacc);
    return -1;
  }
  g_bg[0] = g_bg[1] = g_bg[2] = 0;
  {
    int tt;
    for (tt = 0; tt < nt_max; ++tt) {
      g_bg[0] += bgacc[3 * tt]; g_bg[1] += bgacc[3 * tt + 1]; g_bg[2] += bgacc[3 * tt + 2];
    }
  }
  /* thread sums, then the prologue: det clamp, inverse, sigmoid */
#pragma omp parallel for schedule(static)
  for (g = 0; g < n; ++g) {
    REAL s[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    int tt;
    for (tt = 0; tt < nt_max; ++tt) {
      const REAL* a = acc + nn * 9 * (size_t)tt;
      s[0] += a[3 * g]; s[1] += a[3 * g + 1]; s[2] += a[3 * g + 2];
      s[3] += a[3 * nn + g];
      s[4] += a[4 * nn + 2 * g]; s[5] += a[4 * nn + 2 * g + 1];
      s[6] += a[6 * nn + 3 * g]; s[7] += a[6 * nn + 3 * g + 1]; s[8] += a[6 * nn + 3 * g + 2];
    }
    {
      const REAL c00 = cov2d[4 * g], c01 = cov2d[4 * g + 1], c11 = cov2d[4 * g + 3];
      const REAL draw = c00 * c11 - c01 * c01;
      const REAL det = FN(r_max)(draw, (REAL)1e-6);
      const REAL ct00 = s[0], ct01 = (REAL)2 * s[1], ct11 = s[2];
      const REAL ct_det = -((ct00 * c11 + ct01 * (-c01)) + ct11 * c00) / (det * det) * FN(d_max)(draw, (REAL)1e-6);
      const REAL sg = SIGMOID(opac[g]);
      g_cov2d[4 * g + 0] = ct11 / det + ct_det * c11;
      g_cov2d[4 * g + 1] = -ct01 / det - (REAL)2 * c01 * ct_det;
      g_cov2d[4 * g + 2] = 0;
      g_cov2d[4 * g + 3] = ct00 / det + ct_det * c00;
      g_opac[g] = s[3] * sg * ((REAL)1 - sg);
      g_means2d[2 * g] = s[4];
      g_means2d[2 * g + 1] = s[5];
      g_colors[3 * g] = s[6];
      g_colors[3 * g + 1] = s[7];
      g_colors[3 * g + 2] = s[8];
    }
  }
  free(acc); free(bgacc);
  return 0;
}

/* VJP of eval_sh (sh.py:25-74) for one Gaussian: gsh[k][c] = basis_k * g[c] (0 beyond the
 * degree) and g_d += the cotangent of the view direction d. */
static void FN(sh_vjp)(int K, int deg, const REAL* shi, const REAL* d, const REAL* g_pre, REAL* gsh, REAL* g_d) {
  int c, k;
  /* eval_sh is linear in sh: d/dsh_k = basis_k, obtained by evaluating with unit
   * coefficient vectors; d/d(view dir) by the explicit basis derivatives below. */
  for (k = 0; k < K; ++k) {
    if (k < (deg + 1) * (deg + 1)) {
      REAL unit[48];
      REAL bk;
      memset(unit, 0, sizeof(unit));
      unit[k * 3] = 1;
      bk = FN(eval_sh)(deg, unit, 0, d);
      for (c = 0; c < 3; ++c) gsh[3 * k + c] = bk * g_pre[c];
    } else {
      for (c = 0; c < 3; ++c) gsh[3 * k + c] = 0;
    }
  }
  if (deg > 0) {
    /* directional derivative of sum_c g_pre[c] * eval_sh(c) via the basis gradients */
    const REAL x = d[0], y = d[1], z = d[2];
    const REAL* C2 = FN(C2);
    const REAL* C3 = FN(C3);
    REAL s[16];
    REAL dB[16][3];
    memset(dB, 0, sizeof(dB));
    for (k = 0; k < 16; ++k) s[k] = (k < K && k < (deg + 1) * (deg + 1))
                                        ? (shi[3 * k] * g_pre[0] + shi[3 * k + 1] * g_pre[1]) + shi[3 * k + 2] * g_pre[2]
                                        : (REAL)0;
    dB[1][1] = -FN(C1); dB[2][2] = FN(C1); dB[3][0] = -FN(C1);
    if (deg > 1) {
      dB[4][0] = C2[0] * y; dB[4][1] = C2[0] * x;
      dB[5][1] = C2[1] * z; dB[5][2] = C2[1] * y;
      dB[6][0] = C2[2] * (-2 * x); dB[6][1] = C2[2] * (-2 * y); dB[6][2] = C2[2] * (4 * z);
      dB[7][0] = C2[3] * z; dB[7][2] = C2[3] * x;
      dB[8][0] = C2[4] * (2 * x); dB[8][1] = C2[4] * (-2 * y);
    }
    if (deg > 2) {
      dB[9][0] = C3[0] * 6 * x * y; dB[9][1] = C3[0] * (3 * x * x - 3 * y * y);
      dB[10][0] = C3[1] * y * z; dB[10][1] = C3[1] * x * z; dB[10][2] = C3[1] * x * y;
      dB[11][0] = C3[2] * (-2 * x * y); dB[11][1] = C3[2] * (4 * z * z - x * x - 3 * y * y); dB[11][2] = C3[2] * 8 * y * z;
      dB[12][0] = C3[3] * (-6 * x * z); dB[12][1] = C3[3] * (-6 * y * z); dB[12][2] = C3[3] * (6 * z * z - 3 * x * x - 3 * y * y);
      dB[13][0] = C3[4] * (4 * z * z - 3 * x * x - y * y); dB[13][1] = C3[4] * (-2 * x * y); dB[13][2] = C3[4] * 8 * x * z;
      dB[14][0] = C3[5] * 2 * x * z; dB[14][1] = C3[5] * (-2 * y * z); dB[14][2] = C3[5] * (x * x - y * y);
      dB[15][0] = C3[6] * (3 * x * x - 3 * y * y); dB[15][1] = C3[6] * (-6 * x * y);
    }
    for (k = 0; k < 16; ++k)
      for (c = 0; c < 3; ++c) g_d[c] += s[k] * dB[k][c];
  }
}

int FN(gso_eval_sh)(int64_t n, int K, int deg, const REAL* sh, const REAL* dirs, REAL* out) {
  int64_t i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < n; ++i) {
    int c;
    for (c = 0; c < 3; ++c) out[3 * i + c] = FN(eval_sh)(deg, sh + i * K * 3, c, dirs + 3 * i);
  }
  return 0;
}

int FN(gso_eval_sh_bwd)(int64_t n, int K, int deg, const REAL* sh, const REAL* dirs, const REAL* g_out, REAL* g_sh,
                        REAL* g_dirs) {
  int64_t i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < n; ++i) {
    REAL gd[3] = {0, 0, 0};
    FN(sh_vjp)(K, deg, sh + i * K * 3, dirs + 3 * i, g_out + 3 * i, g_sh + i * K * 3, gd);
    g_dirs[3 * i] = gd[0];
    g_dirs[3 * i + 1] = gd[1];
    g_dirs[3 * i + 2] = gd[2];
  }
  return 0;
}

/* Reverse-mode derivative of gso_preprocess for Gaussian i w.r.t. its mean, scales,
 * quaternion and sh_coeffs given cotangents of means2d, cov2d and colors (radii, valid
 * and depths carry none into the image).  part (may be NULL) receives the Gaussian's
 * share of the W2C cotangent before the camera-centre term: part[3a+b] for W2C[a][b]
 * through the camera-space mean (projection.py:26-27) and W_rot (:52-57), part[9+a] for
 * W2C[a][3], and part[12..14] the cotangent of the view vector m - centre
 * (renderer.py:40-41); the caller adds the centre's share (camera.py:15-21). */
static void FN(pre_bwd_one)(int64_t i, int K, int deg, const REAL* means, const REAL* scales, const REAL* quats,
                            const REAL* sh, const REAL* w2c, REAL fx, REAL fy, const REAL* g_means2d,
                            const REAL* g_cov2d, const REAL* g_colors, REAL* g_means, REAL* g_scales,
                            REAL* g_quats, REAL* g_sh, REAL* part) {
  const REAL* w = w2c;
  {
    FN(proj_t) p;
    REAL v[3], nrm, d[3], g_pre[3], g_d[3] = {0, 0, 0}, g_m[3];
    REAL gx = 0, gy = 0, gz = 0, g_iz, g_iz2, g_zs;
    REAL G[2][2], gT1[2][3], gM2[2][3], gSig[3][3], gJ[2][3], gMm[3][3], gR[3][3], gq[4], qd;
    const REAL* shi = sh + (int64_t)i * K * 3;
    REAL* gsh = g_sh + (int64_t)i * K * 3;
    int a, b, c, k;
    FN(project)(w, means + 3 * i, quats + 4 * i, scales + 3 * i, fx, fy, &p);
    /* colour: clip(eval_sh + 0.5, 0, 1) */
    FN(viewdir)(w, means + 3 * i, v, &nrm, d);
    for (c = 0; c < 3; ++c) {
      const REAL pre = FN(eval_sh)(deg, shi, c, d) + (REAL)0.5;
      const REAL lo = FN(r_max)((REAL)0, pre);
      g_pre[c] = g_colors[3 * i + c] * FN(d_min)(lo, (REAL)1) * FN(d_max)(pre, (REAL)0);
    }
    FN(sh_vjp)(K, deg, shi, d, g_pre, gsh, g_d);
    /* cov2D cotangent; cov2D[1,0] is never read by the renderer */
    G[0][0] = g_cov2d[4 * i]; G[0][1] = g_cov2d[4 * i + 1]; G[1][0] = g_cov2d[4 * i + 2]; G[1][1] = g_cov2d[4 * i + 3];
    /* cov = T1 M2^T, T1 = M2 Sig */
    for (a = 0; a < 2; ++a)
      for (b = 0; b < 3; ++b) {
        gT1[a][b] = G[a][0] * p.M2[0][b] + G[a][1] * p.M2[1][b];
        gM2[a][b] = G[0][a] * p.T1[0][b] + G[1][a] * p.T1[1][b];
      }
    for (a = 0; a < 2; ++a)
      for (b = 0; b < 3; ++b) gM2[a][b] += (gT1[a][0] * p.Sig[b][0] + gT1[a][1] * p.Sig[b][1]) + gT1[a][2] * p.Sig[b][2];
    for (a = 0; a < 3; ++a)
      for (b = 0; b < 3; ++b) gSig[a][b] = p.M2[0][a] * gT1[0][b] + p.M2[1][a] * gT1[1][b];
    /* M2 = J W_rot */
    for (a = 0; a < 2; ++a)
      for (k = 0; k < 3; ++k) gJ[a][k] = (gM2[a][0] * w[k * 4 + 0] + gM2[a][1] * w[k * 4 + 1]) + gM2[a][2] * w[k * 4 + 2];
    g_iz = fx * gJ[0][0] + fy * gJ[1][1];
    g_iz2 = ((-fx) * p.x) * gJ[0][2] + ((-fy) * p.y) * gJ[1][2];
    gx += (-fx) * p.iz2 * gJ[0][2];
    gy += (-fy) * p.iz2 * gJ[1][2];
    g_iz += (REAL)2 * p.iz * g_iz2;
    g_zs = -g_iz / (p.zs * p.zs);
    gz += g_zs * FN(d_max)(p.z, (REAL)0.01);
    /* means2D = fx x / z + cx with the raw depth */
    gx += g_means2d[2 * i] * fx / p.z;
    gy += g_means2d[2 * i + 1] * fy / p.z;
    gz += -(g_means2d[2 * i] * fx * p.x + g_means2d[2 * i + 1] * fy * p.y) / (p.z * p.z);
    for (k = 0; k < 3; ++k) g_m[k] = (w[0 * 4 + k] * gx + w[1 * 4 + k] * gy) + w[2 * 4 + k] * gz;
    if (part != NULL) {
      /* means_cam = W2C[:3,:3] m + W2C[:3,3]; M2 = J W_rot */
      const REAL gp[3] = {gx, gy, gz};
      const REAL J[2][3] = {{fx * p.iz, 0, ((-fx) * p.x) * p.iz2}, {0, fy * p.iz, ((-fy) * p.y) * p.iz2}};
      const REAL* m = means + 3 * i;
      for (a = 0; a < 3; ++a) {
        for (b = 0; b < 3; ++b) part[3 * a + b] += gp[a] * m[b] + (J[0][a] * gM2[0][b] + J[1][a] * gM2[1][b]);
        part[9 + a] += gp[a];
      }
    }
    if (deg > 0) {
      const REAL dg = (d[0] * g_d[0] + d[1] * g_d[1]) + d[2] * g_d[2];
      for (k = 0; k < 3; ++k) {
        const REAL gv = (g_d[k] - d[k] * dg) / nrm;
        g_m[k] += gv;
        if (part != NULL) part[12 + k] += gv;
      }
    }
    for (k = 0; k < 3; ++k) g_means[3 * i + k] = g_m[k];
    /* Sig = Mm Mm^T */
    for (a = 0; a < 3; ++a)
      for (b = 0; b < 3; ++b) {
        REAL acc = 0;
        for (k = 0; k < 3; ++k) acc += (gSig[a][k] + gSig[k][a]) * p.Mm[k][b];
        gMm[a][b] = acc;
      }
    for (b = 0; b < 3; ++b) {
      REAL gs = 0;
      for (a = 0; a < 3; ++a) {
        gR[a][b] = gMm[a][b] * p.s[b];
        gs += gMm[a][b] * p.R[a][b];
      }
      g_scales[3 * i + b] = gs * p.s[b];
    }
    {
      const REAL r = p.qn[0], x = p.qn[1], y = p.qn[2], z = p.qn[3];
      REAL grr = 0, gxx = 0, gyy = 0, gzz = 0;
      gyy += -4 * y * gR[0][0]; gzz += -4 * z * gR[0][0];
      gxx += 2 * y * gR[0][1]; gyy += 2 * x * gR[0][1]; grr += -2 * z * gR[0][1]; gzz += -2 * r * gR[0][1];
      gxx += 2 * z * gR[0][2]; gzz += 2 * x * gR[0][2]; grr += 2 * y * gR[0][2]; gyy += 2 * r * gR[0][2];
      gxx += 2 * y * gR[1][0]; gyy += 2 * x * gR[1][0]; grr += 2 * z * gR[1][0]; gzz += 2 * r * gR[1][0];
      gxx += -4 * x * gR[1][1]; gzz += -4 * z * gR[1][1];
      gyy += 2 * z * gR[1][2]; gzz += 2 * y * gR[1][2]; grr += -2 * x * gR[1][2]; gxx += -2 * r * gR[1][2];
      gxx += 2 * z * gR[2][0]; gzz += 2 * x * gR[2][0]; grr += -2 * y * gR[2][0]; gyy += -2 * r * gR[2][0];
      gyy += 2 * z * gR[2][1]; gzz += 2 * y * gR[2][1]; grr += 2 * x * gR[2][1]; gxx += 2 * r * gR[2][1];
      gxx += -4 * x * gR[2][2]; gyy += -4 * y * gR[2][2];
      gq[0] = grr; gq[1] = gxx; gq[2] = gyy; gq[3] = gzz;
    }
    qd = ((p.qn[0] * gq[0] + p.qn[1] * gq[1]) + p.qn[2] * gq[2]) + p.qn[3] * gq[3];
    for (k = 0; k < 4; ++k) g_quats[4 * i + k] = (gq[k] - p.qn[k] * qd) / p.qnorm;
  }
}

/* Reverse-mode derivative of gso_preprocess w.r.t. means, scales, quaternions and
 * sh_coeffs (outputs overwritten). */
int FN(gso_preprocess_bwd)(int64_t n, int K, int deg, const REAL* means, const REAL* scales, const REAL* quats,
                           const REAL* sh, const REAL* w2c, REAL fx, REAL fy, const REAL* g_means2d,
                           const REAL* g_cov2d, const REAL* g_colors, REAL* g_means, REAL* g_scales, REAL* g_quats,
                           REAL* g_sh) {
  int64_t i;
#pragma omp parallel for schedule(static)
  for (i = 0; i < n; ++i)
    FN(pre_bwd_one)(i, K, deg, means, scales, quats, sh, w2c, fx, fy, g_means2d, g_cov2d, g_colors, g_means,
                    g_scales, g_quats, g_sh, NULL);
  return 0;
}

/* gso_preprocess_bwd plus the W2C cotangent g_w2c[4][4] (row 3 zero: projection.py:27
 * keeps the first three rows of [m, 1] @ W2C^T): the per-Gaussian shares summed per
 * thread, the threads in order, then the camera centre's share
 * (centre = -R^T t, camera.py:15-21: dR[a][b] += t[a] S[b], dt[a] += sum_b R[a][b] S[b],
 * S = the summed view-vector cotangent). */
int FN(gso_preprocess_bwd_w2c)(int64_t n, int K, int deg, const REAL* means, const REAL* scales,
                               const REAL* quats, const REAL* sh, const REAL* w2c, REAL fx, REAL fy,
                               const REAL* g_means2d, const REAL* g_cov2d, const REAL* g_colors, REAL* g_means,
                               REAL* g_scales, REAL* g_quats, REAL* g_sh, REAL* g_w2c) {
  const int nt = omp_get_max_threads();
  REAL* acc = (REAL*)calloc((size_t)nt * 16, sizeof(REAL));
  REAL tot[15];
  int a, b, t;
  if (acc == NULL) return 1;
#pragma omp parallel num_threads(nt)
  {
    REAL* mine = acc + 16 * omp_get_thread_num();
    int64_t j;
#pragma omp for schedule(static)
    for (j = 0; j < n; ++j)
      FN(pre_bwd_one)(j, K, deg, means, scales, quats, sh, w2c, fx, fy, g_means2d, g_cov2d, g_colors, g_means,
                      g_scales, g_quats, g_sh, mine);
  }
  for (a = 0; a < 15; ++a) {
    tot[a] = 0;
    for (t = 0; t < nt; ++t) tot[a] += acc[16 * t + a];
  }
  free(acc);
  for (a = 0; a < 3; ++a) {
    REAL gt = tot[9 + a];
    for (b = 0; b < 3; ++b) {
      g_w2c[4 * a + b] = tot[3 * a + b] + w2c[4 * a + 3] * tot[12 + b];
      gt += w2c[4 * a + b] * tot[12 + b];
    }
    g_w2c[4 * a + 3] = gt;
  }
  for (b = 0; b < 4; ++b) g_w2c[12 + b] = 0;
  return 0;
}

/* jax_gs/training/trainer.py:143-159, the densification statistics of one step:
 * means_cam = [m, 1] @ W2C^T (:145-146), z = max(z_cam, 0.01) (:147),
 * grad_2d_mag = ||dL/dmeans|| * (z / focal) * (W*H*3) (:148-150), focal = (fx+fy)/2,
 * grad_accum += grad_2d_mag (:152), denom += valid & active (:153-154),
 * max_radii = where(valid, max(max_radii, radii), max_radii) (:157-159).
 * active may be NULL (all active). */
int FN(gso_densify)(int64_t n, const REAL* g_means, const REAL* means, const REAL* w2c, REAL focal,
                    REAL pixel_scale, const uint8_t* valid, const uint8_t* active, const REAL* radii,
                    REAL* grad_accum, int32_t* denom, REAL* max_radii) {
  int64_t i;
  for (i = 0; i < n; ++i) {
    const REAL* m = means + 3 * i;
    const REAL* g = g_means + 3 * i;
    const REAL zc = ((m[0] * w2c[8] + m[1] * w2c[9]) + m[2] * w2c[10]) + w2c[11];
    const REAL z = FN(r_max)(zc, (REAL)0.01);
    const REAL nrm = SQRT((g[0] * g[0] + g[1] * g[1]) + g[2] * g[2]);
    const int v = valid[i] != 0;
    const int act = active == NULL || active[i] != 0;
    grad_accum[i] = grad_accum[i] + (nrm * (z / focal)) * pixel_scale;
    denom[i] = denom[i] + ((v && act) ? 1 : 0);
    if (v) max_radii[i] = FN(r_max)(max_radii[i], radii[i]);
  }
  return 0;
}

#undef FN
#undef CAT
#undef CAT2
