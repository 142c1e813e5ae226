"""Pins the CPU oracle against checks that do not restate its own formulas.

Function of the oracle          pinned by
------------------------------  -----------------------------------------------------
gso_expf (float32 exp)          float64 exp, <= 1 ulp over the range the path uses
preprocess: projection/cov/rad  known answers KA1, KA3 (closed form); float64 NumPy
                                J W Sigma W^T J^T with Sigma from a rotation matrix
                                built by scipy.spatial.transform; radius from
                                numpy.linalg.eigvalsh; Sigma symmetric PSD
preprocess: SH colour           scipy.special.sph_harm_y real harmonics (basis =
                                (-1)^m x Condon-Shortley real SH), degrees 0..3
preprocess: camera transform    float64 closed forms under a scipy-rotated, translated
                                W2C: R m + t, J R Sigma R^T J^T + 0.3 I, radii, and the
                                colour from the centre -R^T t (R^T for R, -R t rejected)
tile_interactions               known answer KA2; pure-Python brute force over all
                                256*N slots with Python's stable sorted(); invariants
render_tiles                    KA4, KA5 closed forms (exactly 48 blends in KA5);
                                float64 pure-Python per-pixel brute force; the two
                                reference gathers agree when no clamp triggers
extras                          scenes built to overflow 512 / truncate 4096 /
                                exceed the 16-tile span, with counts known by
                                construction
render_tiles_bwd, preprocess_bwd central finite differences of the float64 oracle;
                                KA3: d image / d opacity = 0 when the 0.99 cap binds;
                                float32 backward within 1e-4 of float64 backward
l1 seed                         closed form sign(d)/count
"""
import math

import numpy as np
import pytest
from scipy.spatial.transform import Rotation

import oracle

F32 = np.float32
C0 = 0.28209479177387814


def _cam(W, H, f, c=None):
    c = (W / 2.0, H / 2.0) if c is None else c
    return dict(W=W, H=H, fx=f, fy=f, cx=c[0], cy=c[1], W2C=np.eye(4, dtype=F32))


def _ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


# ---------------------------------------------------------------- exp
def test_expf_within_one_ulp_of_float64():
    xs = np.concatenate([np.linspace(-87.0, 88.0, 200001, dtype=F32),
                         np.random.default_rng(0).normal(0, 3, 20000).astype(F32),
                         np.linspace(-10.0, 0.0, 20001, dtype=F32)])
    got = np.array([oracle.expf(float(x)) for x in xs[::7]], F32)
    want = np.exp(xs[::7].astype(np.float64)).astype(F32)
    assert _ulp_diff(got, want).max() <= 1
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(-200.0) == 0.0
    assert math.isinf(oracle.expf(100.0))


# ---------------------------------------------------------------- preprocess
def _one(mean, ls, logit=0.0, rgb=(1.0, 1.0, 1.0), q=(1, 0, 0, 0)):
    sh = np.zeros((1, 16, 3), F32)
    sh[0, 0, :] = (np.asarray(rgb, F32) - F32(0.5)) / F32(C0)
    return dict(means=np.array([mean], F32), scales=np.full((1, 3), ls, F32), quaternions=np.array([q], F32),
                opacities=np.array([[logit]], F32), sh_coeffs=sh)


def test_ka1_projection():
    p = _one((0, 0, 5), -3.0)
    pre = oracle.preprocess(p["means"], p["scales"], p["quaternions"], p["sh_coeffs"], np.eye(4), 100, 100, 50.0,
                            50.0, 50.0, 50.0, 0)
    np.testing.assert_array_equal(pre["means2d"][0], [50.0, 50.0])
    assert pre["depths"][0] == 5.0 and pre["valid"][0]
    # closed form: (f/z)^2 exp(-3)^2 + 0.3
    c = (50.0 / 5.0) ** 2 * math.exp(-6.0) + 0.3
    np.testing.assert_allclose(pre["cov2d"][0], [[c, 0], [0, c]], rtol=2e-6, atol=1e-7)
    assert pre["radii"][0] == math.ceil(3 * math.sqrt(c)) == 3


def test_projection_matches_float64_linear_algebra():
    rng = np.random.default_rng(3)
    n = 4000
    means = np.stack([rng.uniform(-1, 1, n), rng.uniform(-1, 1, n), rng.uniform(1, 8, n)], 1).astype(F32)
    scales = rng.normal(-3.0, 0.8, (n, 3)).astype(F32)
    quats = rng.normal(0, 1, (n, 4)).astype(F32)
    sh = np.zeros((n, 1, 3), F32)
    fx, fy, cx, cy = 300.0, 280.0, 160.0, 120.0
    pre = oracle.preprocess(means, scales, quats, sh, np.eye(4), 320, 240, F32(fx), F32(fy), F32(cx), F32(cy), 0)
    q64 = quats.astype(np.float64)
    R = Rotation.from_quat(np.concatenate([q64[:, 1:], q64[:, :1]], 1)).as_matrix()  # scipy: (x,y,z,w)
    S = np.exp(scales.astype(np.float64))
    A = R * S[:, None, :]
    Sig = A @ A.transpose(0, 2, 1)
    x, y, z = (means[:, k].astype(np.float64) for k in range(3))
    J = np.zeros((n, 2, 3))
    J[:, 0, 0] = fx / z
    J[:, 0, 2] = -fx * x / z ** 2
    J[:, 1, 1] = fy / z
    J[:, 1, 2] = -fy * y / z ** 2
    cov = J @ Sig @ J.transpose(0, 2, 1) + 0.3 * np.eye(2)
    np.testing.assert_allclose(pre["cov2d"], cov, rtol=3e-4, atol=1e-5)
    np.testing.assert_allclose(pre["means2d"][:, 0], fx * x / z + cx, rtol=1e-6, atol=1e-4)
    np.testing.assert_allclose(pre["means2d"][:, 1], fy * y / z + cy, rtol=1e-6, atol=1e-4)
    lam = np.linalg.eigvalsh(cov)[:, 1]
    r64 = np.ceil(3 * np.sqrt(lam))
    frac = 3 * np.sqrt(lam) - np.floor(3 * np.sqrt(lam))
    safe = (frac > 1e-4) & (frac < 1 - 1e-4)
    assert safe.mean() > 0.99
    np.testing.assert_array_equal(pre["radii"][safe], r64[safe])
    # Sigma from the float32 path is symmetric positive semi-definite
    assert np.all(np.linalg.eigvalsh(Sig) > -1e-7)


def _camera_closed_form(means, scales, quats, sh, w2c, fx, fy, cx, cy, deg, rot_t=False, centre_rt=False):
    """float64 closed forms of the projection and the colour under a general W2C:
    camera-space mean R m + t (projection.py:26-27), cov2D = J R Sigma R^T J^T + 0.3 I with J
    at the camera-space mean (projection.py:52-57), view direction from the camera centre
    -R^T t (camera.py:15-21, renderer.py:40-41) through scipy's real harmonics.
    rot_t / centre_rt compute the plausible mistakes (R^T for R in the covariance; the centre
    -R t) so that a test can show they fail."""
    n = means.shape[0]
    R = w2c[:3, :3].astype(np.float64)
    t = w2c[:3, 3].astype(np.float64)
    m = means.astype(np.float64)
    pc = m @ R.T + t
    x, y, z = pc[:, 0], pc[:, 1], pc[:, 2]
    q64 = quats.astype(np.float64)
    Rg = Rotation.from_quat(np.concatenate([q64[:, 1:], q64[:, :1]], 1)).as_matrix()
    A = Rg * np.exp(scales.astype(np.float64))[:, None, :]
    Sig = A @ A.transpose(0, 2, 1)
    J = np.zeros((n, 2, 3))
    J[:, 0, 0] = fx / z
    J[:, 0, 2] = -fx * x / z ** 2
    J[:, 1, 1] = fy / z
    J[:, 1, 2] = -fy * y / z ** 2
    Rw = R.T if rot_t else R
    cov = J @ Rw @ Sig @ Rw.T @ J.transpose(0, 2, 1) + 0.3 * np.eye(2)
    m2 = np.stack([fx * x / z + cx, fy * y / z + cy], 1)
    centre = -(R @ t) if centre_rt else -(R.T @ t)
    d = m - centre
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    res = np.zeros((n, 3))
    k = 0
    for l in range(deg + 1):
        for mm in range(-l, l + 1):
            res += _real_sh_no_cs(l, mm, d)[:, None] * sh[:, k, :].astype(np.float64)
            k += 1
    return pc, cov, m2, np.clip(res + 0.5, 0.0, 1.0)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_projection_and_colour_with_rotated_translated_camera(seed):
    """The oracle's forward under a rotated and translated camera (scipy rotation, a
    translation of about half a unit) against the float64 closed forms of
    _camera_closed_form: depth, means2D, cov2D, radii (numpy eigvalsh, away from integer
    boundaries) and the SH-3 colour.  The same comparison rejects R^T in place of R in the
    covariance and the camera centre -R t in place of -R^T t."""
    rng = np.random.default_rng(200 + seed)
    n = 3000
    rot = Rotation.from_rotvec(rng.normal(0.0, 0.5, 3)).as_matrix()
    t = rng.normal(0.0, 0.5, 3)
    w2c = np.eye(4)
    w2c[:3, :3] = rot
    w2c[:3, 3] = t
    w2c = w2c.astype(F32)
    R = w2c[:3, :3].astype(np.float64)
    tt = w2c[:3, 3].astype(np.float64)
    # points in front of the camera, mapped back to the world: m = R^T (p - t)
    z = rng.uniform(1.5, 8.0, n)
    pcam = np.stack([rng.uniform(-0.8, 0.8, n) * z, rng.uniform(-0.6, 0.6, n) * z, z], 1)
    means = ((pcam - tt) @ R).astype(F32)
    scales = rng.normal(-3.0, 0.7, (n, 3)).astype(F32)
    quats = rng.normal(0, 1, (n, 4)).astype(F32)
    sh = rng.normal(0, 0.25, (n, 16, 3)).astype(F32)
    fx, fy, cx, cy = F32(310.0), F32(290.0), F32(200.0), F32(150.0)
    pre = oracle.preprocess(means, scales, quats, sh, w2c, 400, 300, fx, fy, cx, cy, 3)
    pc, cov, m2, col = _camera_closed_form(means, scales, quats, sh, w2c, float(fx), float(fy), float(cx),
                                           float(cy), 3)
    assert pre["valid"].all()
    np.testing.assert_allclose(pre["depths"], pc[:, 2], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(pre["means2d"], m2, rtol=1e-6, atol=2e-4)
    # per Gaussian, relative to the matrix's norm (float32 cancellation in small off-diagonals)
    cerr = np.linalg.norm(pre["cov2d"] - cov, axis=(1, 2)) / np.linalg.norm(cov, axis=(1, 2))
    assert cerr.max() <= 2e-5, cerr.max()
    lam = np.linalg.eigvalsh(cov)[:, 1]
    r = 3.0 * np.sqrt(lam)
    frac = r - np.floor(r)
    safe = (frac > 1e-3) & (frac < 1 - 1e-3)
    assert safe.mean() > 0.99
    np.testing.assert_array_equal(pre["radii"][safe], np.ceil(r[safe]))
    np.testing.assert_allclose(pre["colors"], col, atol=2e-6)
    # the plausible mistakes fail the same bars
    _, cov_t, _, _ = _camera_closed_form(means, scales, quats, sh, w2c, float(fx), float(fy), float(cx), float(cy), 3,
                                         rot_t=True)
    cerr_t = np.linalg.norm(pre["cov2d"] - cov_t, axis=(1, 2)) / np.linalg.norm(cov_t, axis=(1, 2))
    assert cerr_t.max() > 1e-2
    _, _, _, col_rt = _camera_closed_form(means, scales, quats, sh, w2c, float(fx), float(fy), float(cx), float(cy), 3,
                                          centre_rt=True)
    assert not np.allclose(pre["colors"], col_rt, atol=2e-6)


def _real_sh_no_cs(l, m, d):
    from scipy.special import sph_harm_y

    theta = np.arccos(np.clip(d[:, 2], -1, 1))
    phi = np.arctan2(d[:, 1], d[:, 0])
    if m < 0:
        v = math.sqrt(2) * (-1) ** m * sph_harm_y(l, -m, theta, phi).imag
    elif m == 0:
        v = sph_harm_y(l, 0, theta, phi).real
    else:
        v = math.sqrt(2) * (-1) ** m * sph_harm_y(l, m, theta, phi).real
    return (-1) ** m * v


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_sh_colour_matches_scipy_real_harmonics(deg):
    rng = np.random.default_rng(10 + deg)
    n = 300
    means = rng.normal(0, 1, (n, 3)).astype(F32)
    means[:, 2] += 4
    K = 16
    sh = rng.normal(0, 0.2, (n, K, 3)).astype(F32)
    pre = oracle.preprocess(means, np.zeros((n, 3), F32), np.tile(np.array([[1, 0, 0, 0]], F32), (n, 1)), sh,
                            np.eye(4), 64, 64, F32(50), F32(50), F32(32), F32(32), deg)
    d = means.astype(np.float64) / np.linalg.norm(means.astype(np.float64), axis=1, keepdims=True)
    res = np.zeros((n, 3))
    k = 0
    for l in range(deg + 1):
        for m in range(-l, l + 1):
            res += _real_sh_no_cs(l, m, d)[:, None] * sh[:, k, :].astype(np.float64)
            k += 1
    want = np.clip(res + 0.5, 0, 1)
    np.testing.assert_allclose(pre["colors"], want, atol=2e-6)


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_eval_sh_matches_scipy_and_the_render_colour(deg):
    """oracle.eval_sh (sh.py:25-74 on its own) against scipy's real harmonics on
    non-normalised directions' unit vectors, and bit-for-bit against the renderer's colour
    (preprocess: clip(eval_sh + 0.5, 0, 1)) where the clip does not bind."""
    rng = np.random.default_rng(30 + deg)
    n = 200
    d = rng.normal(0, 1, (n, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    sh = rng.normal(0, 0.2, (n, 16, 3)).astype(F32)
    got = oracle.eval_sh(deg, sh, d.astype(F32))
    want = np.zeros((n, 3))
    k = 0
    for l in range(deg + 1):
        for m in range(-l, l + 1):
            want += _real_sh_no_cs(l, m, d.astype(F32).astype(np.float64))[:, None] * sh[:, k, :].astype(np.float64)
            k += 1
    np.testing.assert_allclose(got, want, atol=2e-6)
    means = (d * 4.0).astype(F32)
    pre = oracle.preprocess(means, np.zeros((n, 3), F32), np.tile(np.array([[1, 0, 0, 0]], F32), (n, 1)), sh,
                            np.eye(4), 64, 64, F32(50), F32(50), F32(32), F32(32), deg)
    dirs = means / np.linalg.norm(means.astype(F32), axis=1, keepdims=True).astype(F32)
    col = oracle.eval_sh(deg, sh, dirs) + F32(0.5)
    inside = (col > 0) & (col < 1)
    assert inside.mean() > 0.9
    np.testing.assert_array_equal(pre["colors"][inside], col[inside])


@pytest.mark.parametrize("deg", [1, 2, 3])
def test_eval_sh_vjp_matches_finite_differences(deg):
    """Both cotangents of the float64 eval_sh against central differences, with K = 16 >
    (deg+1)^2 coefficients (the unused ones get 0)."""
    rng = np.random.default_rng(40 + deg)
    n = 6
    d = rng.normal(0, 1, (n, 3))
    sh = rng.normal(0, 0.3, (n, 16, 3))
    g = rng.normal(0, 1, (n, 3))
    g_sh, g_d = oracle.eval_sh_vjp(deg, sh, d, g, dtype=np.float64)
    eps = 1e-6

    def loss(shp, dp):
        return float((oracle.eval_sh(deg, shp, dp, dtype=np.float64) * g).sum())

    for idx in np.ndindex(sh.shape):
        a, b = sh.copy(), sh.copy()
        a[idx] += eps
        b[idx] -= eps
        fd = (loss(a, d) - loss(b, d)) / (2 * eps)
        assert abs(fd - g_sh[idx]) <= 1e-7 + 1e-6 * abs(fd), (idx, fd, g_sh[idx])
    for idx in np.ndindex(d.shape):
        a, b = d.copy(), d.copy()
        a[idx] += eps
        b[idx] -= eps
        fd = (loss(sh, a) - loss(sh, b)) / (2 * eps)
        assert abs(fd - g_d[idx]) <= 1e-7 + 1e-6 * abs(fd), (idx, fd, g_d[idx])
    assert np.all(g_sh[:, (deg + 1) ** 2:] == 0)


# ---------------------------------------------------------------- binning
def test_ka2_tile_interactions():
    st, sg, n = oracle.tile_interactions(np.array([[16, 16], [0, 0]], F32), np.array([4, 2], F32),
                                         np.array([True, True]), np.array([5.0, 10.0], F32), 32, 32)
    assert n == 5 and len(st) == 512
    np.testing.assert_array_equal(st[:5], [0, 0, 1, 2, 3])
    np.testing.assert_array_equal(sg[:5], [0, 1, 0, 0, 0])
    assert np.all(st[5:] == 4)
    np.testing.assert_array_equal(oracle.tile_boundaries(st, 4), [0, 2, 3, 4, 5])


def _brute_bins(means2d, radii, valid, depths, H, W):
    """Pure-Python enumeration of the 256 slots of every Gaussian + Python's stable sort."""
    TX, TY = (W + 15) // 16, (H + 15) // 16
    T = TX * TY
    slots = []
    for i in range(len(radii)):
        mx, my, r = float(means2d[i, 0]), float(means2d[i, 1]), float(radii[i])
        lo_x, hi_x = min(max(mx - r, 0.0), W - 1.0), min(max(mx + r, 0.0), W - 1.0)
        lo_y, hi_y = min(max(my - r, 0.0), H - 1.0), min(max(my + r, 0.0), H - 1.0)
        tx0, tx1, ty0, ty1 = int(lo_x // 16), int(hi_x // 16), int(lo_y // 16), int(hi_y // 16)
        on = (mx + r > 0) and (mx - r < W) and (my + r > 0) and (my - r < H)
        v = bool(valid[i]) and on and tx1 >= tx0 and ty1 >= ty0
        zbits = int(np.array([depths[i]], F32).view(np.int32)[0])
        dq = zbits >> 18
        for oy in range(16):
            for ox in range(16):
                ax, ay = tx0 + ox, ty0 + oy
                tile = ay * TX + ax if (v and ax <= tx1 and ay <= ty1) else T
                key = ((tile << 13) | dq)
                key = key - (1 << 32) if key >= (1 << 31) else key
                slots.append((key, i))
    order = sorted(range(len(slots)), key=lambda j: slots[j][0])  # stable
    return [slots[j][0] >> 13 for j in order], [slots[j][1] for j in order]


def test_tile_interactions_brute_force():
    rng = np.random.default_rng(5)
    n = 40
    W, H = 70, 50
    means2d = rng.uniform(-20, 90, (n, 2)).astype(F32)
    radii = np.ceil(rng.uniform(0, 40, n)).astype(F32)
    radii[:3] = 400  # spans wider than 16 tiles are truncated
    valid = rng.uniform(0, 1, n) < 0.85
    depths = rng.uniform(0.02, 9, n).astype(F32)
    depths[5] = depths[6]  # equal depth bucket: ties resolve by Gaussian id
    depths[7] = -1.0       # negative depth: its 256 slots sort first with tile -1
    valid[7] = False
    st, sg, cnt = oracle.tile_interactions(means2d, radii, valid, depths, H, W)
    bt, bg = _brute_bins(means2d, radii, valid, depths, H, W)
    np.testing.assert_array_equal(st, bt)
    np.testing.assert_array_equal(sg, bg)
    T = ((W + 15) // 16) * ((H + 15) // 16)
    assert cnt == int(np.sum((np.asarray(bt) >= 0) & (np.asarray(bt) < T)))
    assert np.sum(np.asarray(bt) == -1) == 256


# ---------------------------------------------------------------- compositing
def _brute_render(means2d, cov2d, opac, colors, st, sg, H, W, bg):
    """float64, per pixel, straight from the definition (first min(count,4096) entries)."""
    TX = (W + 15) // 16
    T = TX * ((H + 15) // 16)
    img = np.zeros((H, W, 3))
    b = np.searchsorted(st, np.arange(T + 1), side="left")
    for t in range(T):
        ids = sg[b[t]:b[t + 1]][:4096]
        tx, ty = t % TX, t // TX
        for ly in range(16):
            for lx in range(16):
                X, Y = tx * 16 + lx, ty * 16 + ly
                if X >= W or Y >= H:
                    continue
                if len(ids) == 0:
                    img[Y, X] = bg
                    continue
                C = np.zeros(3)
                Tr = 1.0
                for g in ids:
                    if Tr <= 1e-4:
                        break
                    c = cov2d[g].astype(np.float64)
                    det = max(c[0, 0] * c[1, 1] - c[0, 1] ** 2, 1e-6)
                    inv = np.array([[c[1, 1], -c[0, 1]], [-c[0, 1], c[0, 0]]]) / det
                    d = np.array([X + 0.5, Y + 0.5]) - means2d[g]
                    pw = -0.5 * d @ inv @ d
                    if pw <= -10:
                        continue
                    a = min(0.99, math.exp(pw) / (1 + math.exp(-float(opac[g, 0]))))
                    C += a * Tr * colors[g]
                    Tr *= 1 - a
                img[Y, X] = C + Tr * bg
    return img


def test_render_tiles_brute_force():
    rng = np.random.default_rng(8)
    n = 30
    W, H = 40, 36
    pre_m = rng.uniform(0, 40, (n, 2)).astype(F32)
    A = rng.normal(0, 3, (n, 2, 2))
    cov = (A @ A.transpose(0, 2, 1) + 0.3 * np.eye(2)).astype(F32)
    opac = rng.normal(0, 2, (n, 1)).astype(F32)
    col = rng.uniform(0, 1, (n, 3)).astype(F32)
    radii = np.ceil(3 * np.sqrt(np.linalg.eigvalsh(cov.astype(np.float64))[:, 1])).astype(F32)
    depths = rng.uniform(1, 5, n).astype(F32)
    st, sg, _ = oracle.tile_interactions(pre_m, radii, np.ones(n, bool), depths, H, W)
    bg = np.array([0.1, 0.2, 0.3], F32)
    img, fT, nc = oracle.render_tiles(pre_m, cov, opac, col, st, sg, H, W, bg)
    ref = _brute_render(pre_m, cov, opac, col, st, sg, H, W, bg.astype(np.float64))
    np.testing.assert_allclose(img, ref, atol=2e-5)
    img_tpu, _, _ = oracle.render_tiles(pre_m, cov, opac, col, st, sg, H, W, bg, tpu_gather=True)
    np.testing.assert_allclose(img_tpu, img, atol=2e-6)
    assert np.all(np.diff(fT.ravel()) == np.diff(fT.ravel()))  # finite
    assert fT.min() > 0 and fT.max() <= 1


def test_ka4_single_gaussian():
    img, _, _ = oracle.render_tiles(np.array([[16, 16]], F32), np.array([[[10, 0], [0, 10]]], F32),
                                    np.array([[10.0]], F32), np.array([[1, 0, 0]], F32),
                                    np.array([0, 1, 2, 3], np.int32), np.zeros(4, np.int32), 32, 32)
    want = math.exp(-0.5 * 0.5 / 10) * (1 / (1 + math.exp(-10)))
    np.testing.assert_allclose(img[16, 16], [want, 0, 0], rtol=2e-6, atol=1e-7)


def test_ka5_chunked_gated_composite():
    N = 520
    means2d = np.tile(np.array([[8, 8]], F32), (N, 1))
    cov = np.tile(np.array([[[6, 0], [0, 6]]], F32), (N, 1, 1))
    op = np.full((N, 1), -1.5, F32)
    col = np.stack([np.linspace(0, 1, N, dtype=F32), np.linspace(1, 0, N, dtype=F32), np.zeros(N, F32)], -1)
    img, fT, nc = oracle.render_tiles(means2d, cov, op, col, np.zeros(N, np.int32), np.arange(N, dtype=np.int32),
                                      16, 16)
    a = math.exp(-0.5 * 0.5 / 6) / (1 + math.exp(1.5))
    assert abs(a - 0.17498064) < 1e-7
    k = 0
    Tr = 1.0
    C = np.zeros(3)
    while Tr > 1e-4:
        C += a * Tr * col[k].astype(np.float64)
        Tr *= 1 - a
        k += 1
    assert k == 48 and nc[8, 8] == 48
    np.testing.assert_allclose(img[8, 8], C, atol=2e-6)
    np.testing.assert_allclose(img[8, 8], [0.0090747, 0.9908275, 0.0], atol=1e-6)


def test_extras_overflow_truncation_and_span_cap():
    n = 4200
    W = H = 64
    means2d = np.tile(np.array([[8.0, 8.0]], F32), (n, 1))
    radii = np.full(n, 2.0, F32)           # one tile each
    radii[:2] = 600.0                      # spans over 16 tiles (image is 4x4 tiles: no cap)
    depths = np.linspace(1, 3, n).astype(F32)
    pre = dict(means2d=means2d, radii=radii, valid=np.ones(n, bool), depths=depths)
    st, sg, cnt = oracle.tile_interactions(means2d, radii, pre["valid"], depths, H, W)
    assert cnt == (n - 2) + 2 * 16
    ex = oracle.extras_from(pre, st, cnt, H, W)
    assert ex["max_interactions_per_tile"] == n
    assert ex["truncated_tiles"] == 1 and ex["truncated_interactions"] == n - 4096
    assert ex["overflow_tiles"] == 1 and ex["overflow_interactions"] == n - 512
    assert ex["radius_cap_violations"] == 0
    # a 30x30-tile image: the two wide Gaussians exceed the 16-tile span
    st, sg, cnt = oracle.tile_interactions(means2d, radii, pre["valid"], depths, 480, 480)
    assert cnt == (n - 2) + 2 * 16 * 16
    ex = oracle.extras_from(pre, st, cnt, 480, 480)
    assert ex["radius_cap_violations"] == 2


# ---------------------------------------------------------------- backward
def _tiny_scene(seed, n=12, W=40, H=32, deg=3):
    rng = np.random.default_rng(seed)
    means = np.stack([rng.uniform(-0.6, 0.6, n), rng.uniform(-0.5, 0.5, n), rng.uniform(2.5, 4, n)], 1)
    sh = np.zeros((n, 16, 3))
    sh[:, 0, :] = (rng.uniform(0.2, 0.8, (n, 3)) - 0.5) / C0
    sh[:, 1:, :] = rng.normal(0, 0.05, (n, 15, 3))
    params = dict(means=means, scales=rng.normal(-2.3, 0.2, (n, 3)), quaternions=rng.normal(0, 1, (n, 4)),
                  opacities=rng.normal(0, 1, (n, 1)), sh_coeffs=sh)
    return params, _cam(W, H, 30.0), deg


def _fd_check(params, cam, deg, seed_img, dtype=np.float64, eps=1e-6, sample=8):
    img, _, res = oracle.render(params, cam, sh_degree=deg, dtype=dtype)
    g = oracle.render_vjp(params, cam, res, seed_img, sh_degree=deg, dtype=dtype)
    rng = np.random.default_rng(1)

    def loss(p):
        im, _, _ = oracle.render(p, cam, sh_degree=deg, dtype=dtype)
        return float((im * seed_img).sum())

    for f in ("means", "scales", "quaternions", "opacities", "sh_coeffs"):
        flat = params[f].reshape(-1)
        idx = rng.choice(flat.size, size=min(sample, flat.size), replace=False)
        if f == "sh_coeffs":
            idx = np.concatenate([idx, [0, 3 * 5 + 1, 3 * 15 + 2]])
        for i in idx:
            pp = {k: v.copy() for k, v in params.items()}
            pp[f].reshape(-1)[i] += eps
            lp = loss(pp)
            pp[f].reshape(-1)[i] -= 2 * eps
            lm = loss(pp)
            fd = (lp - lm) / (2 * eps)
            an = g[f].reshape(-1)[i]
            assert abs(fd - an) <= 1e-5 * max(1.0, abs(fd)) + 1e-7, (f, i, fd, an)
    return g


@pytest.mark.parametrize("seed", [0, 1])
def test_backward_matches_finite_differences(seed):
    params, cam, deg = _tiny_scene(seed)
    rng = np.random.default_rng(100 + seed)
    seed_img = rng.normal(0, 1, (cam["H"], cam["W"], 3))
    _fd_check(params, cam, deg, seed_img)


def _oblique_w2c():
    """A rotation by 0.2 rad about an oblique axis (Rodrigues) and a translation, so that
    every entry of W2C's first three rows enters the projection."""
    ax = np.array([0.3, -0.5, 0.8])
    ax /= np.linalg.norm(ax)
    Kx = np.array([[0, -ax[2], ax[1]], [ax[2], 0, -ax[0]], [-ax[1], ax[0], 0]])
    w = np.eye(4)
    w[:3, :3] = np.eye(3) + math.sin(0.2) * Kx + (1 - math.cos(0.2)) * Kx @ Kx
    w[:3, 3] = [0.1, -0.05, 0.3]
    return w


@pytest.mark.parametrize("seed", [0, 1])
def test_w2c_cotangent_matches_finite_differences(seed):
    """dL/dW2C of the float64 oracle (projection.py:26-57 through the camera-space mean and
    W_rot, renderer.py:40-41 and camera.py:15-21 through the view direction) against
    central differences of the rendered loss in all 16 entries (row 3 never enters)."""
    params, cam, deg = _tiny_scene(seed)
    cam = dict(cam, W2C=_oblique_w2c())
    seed_img = np.random.default_rng(200 + seed).normal(0, 1, (cam["H"], cam["W"], 3))
    _, _, res = oracle.render(params, cam, sh_degree=deg, dtype=np.float64)
    g = oracle.render_vjp(params, cam, res, seed_img, sh_degree=deg, dtype=np.float64)["W2C"]
    eps = 1e-6
    for a in range(4):
        for b in range(4):
            lv = []
            for sgn in (1, -1):
                w = cam["W2C"].copy()
                w[a, b] += sgn * eps
                im, _, _ = oracle.render(params, dict(cam, W2C=w), sh_degree=deg, dtype=np.float64)
                lv.append(float((im * seed_img).sum()))
            fd = (lv[0] - lv[1]) / (2 * eps)
            assert abs(fd - g[a, b]) <= 1e-5 * max(1.0, abs(fd)) + 1e-7, (a, b, fd, g[a, b])
    assert np.all(g[3] == 0) and np.abs(g[:3]).min() > 0


def test_float32_backward_close_to_float64():
    params, cam, deg = _tiny_scene(4)
    seed_img = np.random.default_rng(3).normal(0, 1, (cam["H"], cam["W"], 3))
    p32 = {k: v.astype(F32) for k, v in params.items()}
    p64 = {k: v.astype(F32).astype(np.float64) for k, v in params.items()}
    _, _, r32 = oracle.render(p32, cam, sh_degree=deg)
    g32 = oracle.render_vjp(p32, cam, r32, seed_img.astype(F32), sh_degree=deg)
    _, _, r64 = oracle.render(p64, cam, sh_degree=deg, dtype=np.float64)
    g64 = oracle.render_vjp(p64, cam, r64, seed_img, sh_degree=deg, dtype=np.float64)
    for f in ("means", "scales", "quaternions", "opacities", "sh_coeffs"):
        rel = np.linalg.norm(g32[f] - g64[f]) / np.linalg.norm(g64[f])
        assert rel < 1e-4, (f, rel)


def test_ka3_capped_alpha_has_zero_opacity_gradient():
    p = _one((0, 0, 5), -1.0, logit=10.0, rgb=(1, 0, 0))
    cam = _cam(64, 64, 100.0, (32.0, 32.0))
    img, ex, res = oracle.render(p, cam)
    c = (100.0 / 5.0) ** 2 * math.exp(-2.0) + 0.3
    np.testing.assert_allclose(res["pre"]["cov2d"][0, 0, 0], c, rtol=2e-6)
    assert res["pre"]["radii"][0] == 23
    np.testing.assert_allclose(img[32, 32], [0.99, 0, 0], atol=1e-6)
    g = np.zeros_like(img)
    g[32, 32, 0] = 1
    gr = oracle.render_vjp(p, cam, res, g)
    assert gr["opacities"][0, 0] == 0.0
    # one pixel off the centre the cap does not bind: gradient is positive
    g2 = np.zeros_like(img)
    g2[32, 40, 0] = 1
    assert oracle.render_vjp(p, cam, res, g2)["opacities"][0, 0] > 0


def test_l1_seed_closed_form():
    a = np.array([[[0.5, 0.2, 0.7]]], F32)
    b = np.array([[[0.5, 0.9, 0.1]]], F32)
    loss, g = oracle.l1_loss_and_grad(a, b)
    np.testing.assert_allclose(loss, (0 + 0.7 + 0.6) / 3, rtol=1e-6)
    np.testing.assert_array_equal(g, np.array([[[0, -1, 1]]], F32) * F32(1 / 3))


def test_densify_closed_form():
    """trainer.py:143-159 on hand-computable cases: z/focal = 1/64, |g| = 5, W*H*3 = 192
    give exactly 15; a Gaussian behind the camera uses z = 0.01; denom counts valid and
    active only; max_radii moves only for valid Gaussians."""
    w2c = np.eye(4, dtype=np.float32)
    w2c[2, 3] = 1.0  # z_cam = z + 1
    means = np.array([[0.5, -2.0, 3.0], [1.0, 1.0, -4.0], [0.0, 0.0, 3.0], [2.0, 2.0, 3.0]], np.float32)
    g = np.array([[3.0, 4.0, 0.0], [0.0, 0.0, 5.0], [0.0, 0.0, 0.0], [4.0, 0.0, 3.0]], np.float32)
    valid = np.array([1, 1, 0, 1], np.uint8)
    active = np.array([1, 1, 1, 0], np.uint8)
    radii = np.array([7.0, 2.0, 50.0, 9.0], np.float32)
    ga0 = np.array([1.0, 0.0, 0.5, 0.0], np.float32)
    de0 = np.array([2, 0, 1, 3], np.int32)
    mr0 = np.array([3.0, 4.0, 5.0, 6.0], np.float32)
    ga, de, mr = oracle.densify(g, means, w2c, 200.0, 312.0, 8, 8, valid, radii, ga0, de0, mr0, active=active)
    assert ga[0] == 1.0 + 15.0 and ga[3] == 15.0  # z = 4, focal = 256
    assert abs(ga[1] - 5.0 * (0.01 / 256.0) * 192.0) <= 1e-7  # z_cam = -3 -> 0.01
    assert ga[2] == 0.5
    np.testing.assert_array_equal(de, [3, 1, 1, 3])
    np.testing.assert_array_equal(mr, [7.0, 4.0, 5.0, 9.0])


def test_densify_float32_matches_float64():
    rng = np.random.default_rng(4)
    n = 500
    means = rng.normal(0, 2, (n, 3)).astype(np.float32)
    g = rng.normal(0, 1e-3, (n, 3)).astype(np.float32)
    w2c = np.eye(4, dtype=np.float32)
    w2c[:3, 3] = [0.1, -0.2, 4.0]
    valid = (rng.uniform(size=n) < 0.8).astype(np.uint8)
    radii = np.ceil(rng.uniform(0, 30, n)).astype(np.float32)
    z = np.zeros(n, np.float32)
    out32 = oracle.densify(g, means, w2c, 500.0, 510.0, 64, 48, valid, radii, z, np.zeros(n, np.int32), z)
    out64 = oracle.densify(g, means, w2c, 500.0, 510.0, 64, 48, valid, radii, z, np.zeros(n, np.int32), z,
                           dtype=np.float64)
    np.testing.assert_allclose(out32[0], out64[0], rtol=1e-5)
    np.testing.assert_array_equal(out32[1], out64[1])
    np.testing.assert_array_equal(out32[2], out64[2])


# ---------------------------------------------------------------------------------------
# SSIM restatement (losses.py:16-75)
def test_ssim_window_is_the_normalised_gaussian():
    from scipy.signal.windows import gaussian

    w = oracle.ssim_window(dtype=np.float64)
    g = gaussian(11, std=1.5)
    np.testing.assert_allclose(w, g / g.sum(), rtol=1e-14)


def test_ssim_blur_matches_scipy():
    """Separable 'SAME' zero-padded correlation = scipy's correlate1d twice = a 2-D
    convolution with the outer product of the taps."""
    from scipy.ndimage import correlate1d
    from scipy.signal import convolve2d

    rng = np.random.default_rng(1)
    img = rng.normal(size=(12, 17, 3))
    w = oracle.ssim_window(dtype=np.float64)
    got = oracle.ssim_blur(img, w)
    want = correlate1d(correlate1d(img, w, axis=0, mode="constant"), w, axis=1, mode="constant")
    np.testing.assert_allclose(got, want, atol=1e-13)
    for c in range(3):
        np.testing.assert_allclose(got[..., c], convolve2d(img[..., c], np.outer(w, w), mode="same"), atol=1e-13)


@pytest.mark.parametrize("L", [1, 4, 7, 10, 15])
def test_ssim_blur_any_window_is_xla_same_correlation(L):
    """Any window size: XLA's 'SAME' padding (TensorFlow's documented rule: L - 1 padded
    values, (L - 1) // 2 of them before) and a 'valid' correlation of the padded image
    (scipy.signal.correlate), per axis; the adjoint is the transposed matrix."""
    from scipy.signal import correlate

    rng = np.random.default_rng(L)
    img = rng.normal(size=(12, 17, 2))
    w = oracle.ssim_window(L, dtype=np.float64)
    lo = (L - 1) // 2
    pad = np.pad(img, ((lo, L - 1 - lo), (lo, L - 1 - lo), (0, 0)))
    want = np.stack([correlate(pad[..., c], np.outer(w, w), mode="valid") for c in range(2)], -1)
    np.testing.assert_allclose(oracle.ssim_blur(img, w), want, atol=1e-13)
    # adjoint: <blur(a), b> = <a, blur^T(b)>
    b = rng.normal(size=img.shape)
    lhs = (oracle.ssim_blur(img, w) * b).sum()
    rhs = (img * oracle.ssim_blur(b, w, adjoint=True)).sum()
    assert abs(lhs - rhs) <= 1e-12 * abs(lhs)


@pytest.mark.parametrize("L", [4, 7])
def test_ssim_any_window_vjp_and_fixture(L):
    """The reference's test_training.py:21-38 properties at another window size, and the
    VJP against central differences (even L: the off-centre window)."""
    rng = np.random.default_rng(20 + L)
    target = rng.uniform(0, 1, (16, 18, 3))
    pred = target + 0.1 * rng.uniform(0, 1, target.shape)
    s = oracle.ssim(pred, target, window_size=L)
    assert 0.0 <= s <= 1.0 and np.isclose(oracle.ssim(target, target, window_size=L), 1.0)
    x = rng.uniform(0, 1, (7, 9, 2))
    y = rng.uniform(0, 1, (7, 9, 2))
    g = oracle.ssim_vjp(x, y, 1.0, window_size=L)
    num = np.zeros_like(x)
    eps = 1e-6
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += eps
        xm[idx] -= eps
        num[idx] = (oracle.ssim(xp, y, window_size=L) - oracle.ssim(xm, y, window_size=L)) / (2 * eps)
    assert np.linalg.norm(num - g) / np.linalg.norm(num) < 1e-6


def test_ssim_reference_fixture():
    """test_training.py:21-38: bounds, d_ssim = (1 - ssim) / 2, perfect match."""
    rng = np.random.default_rng(0)
    target = rng.uniform(0, 1, (32, 32, 3))
    pred = target + 0.1 * rng.uniform(0, 1, target.shape)
    s = oracle.ssim(pred, target)
    assert 0.0 <= s <= 1.0
    assert 0.0 <= oracle.d_ssim_loss(pred, target) <= 1.0
    assert np.isclose(oracle.d_ssim_loss(pred, target), (1.0 - s) / 2.0)
    assert np.isclose(oracle.ssim(target, target), 1.0)
    assert np.isclose(oracle.d_ssim_loss(target, target), 0.0)


def test_ssim_constant_images_closed_form():
    """Constant images a and b: away from the zero-padded border (>= 5 pixels) the means
    are a and b and the variances 0, so the map is (2ab + C1) / (a^2 + b^2 + C1)."""
    a, b = 0.3, 0.7
    x = np.full((24, 26, 2), a)
    y = np.full((24, 26, 2), b)
    m = oracle.ssim_map(x, y)
    want = (2 * a * b + oracle.SSIM_C1) / (a * a + b * b + oracle.SSIM_C1)
    np.testing.assert_allclose(m[5:-5, 5:-5], want, rtol=1e-12)
    assert np.all(m[:5] != want)  # the border sees the zero padding


def test_ssim_vjp_matches_finite_differences():
    rng = np.random.default_rng(2)
    x = rng.uniform(0, 1, (9, 13, 2))
    y = rng.uniform(0, 1, (9, 13, 2))
    g = oracle.ssim_vjp(x, y, 1.0)
    num = np.zeros_like(x)
    eps = 1e-6
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += eps
        xm[idx] -= eps
        num[idx] = (oracle.ssim(xp, y) - oracle.ssim(xm, y)) / (2 * eps)
    assert np.linalg.norm(num - g) / np.linalg.norm(num) < 1e-6
    # the cotangent scales the result; d_ssim's cotangent is -1/2 of ssim's
    np.testing.assert_allclose(oracle.ssim_vjp(x, y, 3.0), 3.0 * g, rtol=1e-12)
    np.testing.assert_allclose(oracle.d_ssim_vjp(x, y, 1.0), -0.5 * g, rtol=1e-12)


def test_ssim_float32_matches_float64():
    rng = np.random.default_rng(3)
    x = rng.uniform(0, 1, (40, 50, 3)).astype(np.float32)
    y = rng.uniform(0, 1, (40, 50, 3)).astype(np.float32)
    assert abs(oracle.ssim(x, y, np.float32) - oracle.ssim(x, y, np.float64)) < 1e-6
    g32 = oracle.ssim_vjp(x, y, 1.0, np.float32)
    g64 = oracle.ssim_vjp(x, y, 1.0, np.float64)
    assert np.linalg.norm(g32 - g64) / np.linalg.norm(g64) < 1e-4


def test_mse_closed_form():
    """test_training.py:9-19: mean of (0.1^2, 0.1^2, 0) = 0.00666..."""
    pred = np.array([1.0, 2.0, 3.0], np.float32)
    target = np.array([1.1, 1.9, 3.0], np.float32)
    loss, seed = oracle.mse_loss_and_grad(pred, target)
    assert np.isclose(loss, 0.00666667, atol=1e-7)
    np.testing.assert_allclose(seed, 2 * (pred - target) / 3, rtol=1e-6)


# ---------------------------------------------------------------------------------------
# Optimizer restatement (optax.adam, trainer.py:44-53 mask)
def test_adam_first_step_and_constant_gradient_closed_forms():
    """With zero moments, or after t steps of one constant gradient g, the bias-corrected
    moments are g and g^2, so every update is -lr g / (|g| + eps)."""
    rng = np.random.default_rng(0)
    g = rng.normal(size=(50, 3)).astype(np.float32)
    p = rng.normal(size=(50, 3)).astype(np.float32)
    mu = np.zeros_like(p)
    nu = np.zeros_like(p)
    lr = 0.005
    want = -lr * g.astype(np.float64) / (np.abs(g.astype(np.float64)) + 1e-8)
    q = p.copy()
    for t in range(5):
        q_new, mu, nu = oracle.adam_step(q, g, mu, nu, t, lr)
        np.testing.assert_allclose(q_new.astype(np.float64) - q, want, rtol=2e-3, atol=1e-9)
        q = q_new
    np.testing.assert_allclose(mu, g * (1 - 0.9 ** 5), rtol=1e-5)
    np.testing.assert_allclose(nu, g * g * (1 - 0.999 ** 5), rtol=1e-4)


def test_adam_mask_keeps_inactive_rows_but_moves_their_moments():
    rng = np.random.default_rng(1)
    p = rng.normal(size=(8, 4)).astype(np.float32)
    g = rng.normal(size=(8, 4)).astype(np.float32)
    active = np.array([1, 0, 1, 1, 0, 0, 1, 0], bool)
    q, mu, nu = oracle.adam_step(p, g, np.zeros_like(p), np.zeros_like(p), 0, 0.001, active)
    np.testing.assert_array_equal(q[~active], p[~active])
    assert np.all(q[active] != p[active])
    np.testing.assert_allclose(mu, 0.1 * g, rtol=1e-6)


def test_exponential_decay_schedule():
    """train.py:127-135: lr(0) = init, lr(T) = end, lr(T/2) = sqrt(init * end)."""
    init, end, T = 0.00016 * 3.0 * 2.5, 0.0000016 * 3.0 * 2.5, 30000
    s = oracle.exponential_decay(init, T, end / init)
    assert s(0) == np.float32(init)
    assert np.isclose(s(T), end, rtol=1e-5)
    assert np.isclose(s(T // 2), np.sqrt(init * end), rtol=1e-5)


# ---------------------------------------------------------------------------------------
# densify_and_prune restatement (density.py:98-211)
def _den_state(M, K=1):
    f = np.float32
    return {"means": np.zeros((M, 3), f), "scales": np.full((M, 3), np.log(0.02), f),
            "quaternions": np.tile(np.array([1, 0, 0, 0], f), (M, 1)), "opacities": np.zeros((M, 1), f),
            "sh_coeffs": np.zeros((M, K, 3), f), "active": np.zeros(M, bool), "grad_accum": np.zeros(M, f),
            "denom": np.zeros(M, np.int32), "max_radii": np.zeros(M, f), "moments": {}}


def test_densify_hand_built_case():
    """Slots 0-3 active, 4-7 empty; 1 is transparent (pruned), 2 has a high average
    gradient and a small scale (cloned), 3 a high gradient and a scale above 1% of the
    extent (split).  Empty slots after pruning are 1, 4, 5, 6, 7: slot 1 takes the
    clone of 2, slot 4 the split copy of 3."""
    s = _den_state(8)
    s["active"][:4] = True
    s["means"][:] = np.arange(24, dtype=np.float32).reshape(8, 3)
    s["opacities"][1, 0] = -10.0
    s["grad_accum"][2], s["denom"][2] = 0.001, 2        # avg 5e-4 >= 2e-4
    s["grad_accum"][3], s["denom"][3] = 0.003, 3        # avg 1e-3
    s["scales"][3] = np.log(0.2)                        # 0.05 < 0.2 < 0.5 (extent 5)
    s["sh_coeffs"][:, 0, 0] = np.arange(8)
    s["moments"] = {"mu": np.arange(8, dtype=np.float32)[:, None] * np.ones((1, 3), np.float32)}
    noise = np.random.default_rng(0).normal(size=(8, 3)).astype(np.float32)
    out, c = oracle.densify_and_prune(s, noise, extent=5.0)
    assert (c["clones"], c["splits"], c["pruned"], c["available"]) == (1, 1, 1, 5)
    assert list(np.flatnonzero(out["active"])) == [0, 1, 2, 3, 4]
    assert list(c["gather"]) == [0, 2, 2, 3, 3, 5, 6, 7]
    np.testing.assert_array_equal(out["means"][1], s["means"][2])
    assert out["sh_coeffs"][1, 0, 0] == 2 and out["sh_coeffs"][4, 0, 0] == 3
    np.testing.assert_array_equal(out["moments"]["mu"][[1, 4], 0], [2, 3])
    s_new = np.float32(np.float32(np.log(0.2)) - np.float32(np.log(1.6)))
    for slot in (3, 4):
        np.testing.assert_array_equal(out["scales"][slot], np.full(3, s_new, np.float32))
        want = s["means"][3] + noise[slot] * oracle.expf_array(np.full(3, s_new, np.float32))
        np.testing.assert_allclose(out["means"][slot], want, rtol=1e-6)
    assert not out["grad_accum"].any() and not out["denom"].any()


def test_densify_capacity_and_switch():
    """Nothing is added when the new Gaussians do not fit or densify_enabled is False;
    pruning (opacity, world size, screen size) still applies."""
    s = _den_state(6)
    s["active"][:] = True
    s["grad_accum"][:3], s["denom"][:3] = 0.01, 1        # three clone candidates, no room
    s["max_radii"][5] = 600.0                           # pruned by screen size
    s["scales"][4] = np.log(0.6)                        # pruned by world size (> 0.5)
    out, c = oracle.densify_and_prune(s, np.zeros((6, 3), np.float32), extent=5.0)
    assert (c["clones"], c["splits"], c["pruned"], c["available"]) == (0, 0, 2, 2)
    assert list(np.flatnonzero(out["active"])) == [0, 1, 2, 3]
    s["max_radii"][5] = 0.0
    s["scales"][4] = np.log(0.02)
    s["active"][4:] = False
    out, c = oracle.densify_and_prune(s, np.zeros((6, 3), np.float32), densify_enabled=False, extent=5.0)
    assert (c["clones"], c["splits"]) == (0, 0) and list(np.flatnonzero(out["active"])) == [0, 1, 2, 3]


def test_densify_random_invariants():
    rng = np.random.default_rng(5)
    M = 500
    s = _den_state(M, K=4)
    s["active"] = rng.uniform(size=M) < 0.6
    s["opacities"][:, 0] = rng.normal(0, 3, M)
    s["scales"][:] = np.log(rng.uniform(0.005, 0.3, (M, 3)))
    s["grad_accum"][:] = rng.uniform(0, 0.002, M)
    s["denom"][:] = rng.integers(0, 5, M)
    s["means"][:] = rng.normal(size=(M, 3))
    s["sh_coeffs"][:] = rng.normal(size=(M, 4, 3))
    noise = rng.normal(size=(M, 3)).astype(np.float32)
    out, c = oracle.densify_and_prune(s, noise, extent=5.0)
    added = c["clones"] + c["splits"]
    assert added > 0
    after = int(s["active"].sum()) - c["pruned"]
    assert int(out["active"].sum()) == after + added
    moved = np.flatnonzero(c["gather"] != np.arange(M))
    assert len(moved) == added and not s["active"][moved].all()
    for slot in moved:   # copies carry their source's SH and quaternion exactly
        np.testing.assert_array_equal(out["sh_coeffs"][slot], s["sh_coeffs"][c["gather"][slot]])


# ---------------------------------------------------------------------------------------
# PLY bytes (ply.py:6-123)
def test_ply_bytes_layout():
    """Header lines and the byte offset of every property: value j of vertex v sits at
    header + (62 v + j) * 4, little-endian float32, f_rest_i = sh[1 + i // 3][i % 3]."""
    n = 3
    v = np.arange(n, dtype=np.float32)[:, None]
    means = 1000 * v + np.arange(3, dtype=np.float32)
    sh = (1000 * v[:, :, None] + 100 + np.arange(48, dtype=np.float32).reshape(1, 16, 3)).astype(np.float32)
    opac = 1000 * v + 200
    scales = 1000 * v + 300 + np.arange(3, dtype=np.float32)
    quats = 1000 * v + 400 + np.arange(4, dtype=np.float32)
    b = oracle.ply_bytes(means, scales, quats, opac, sh)
    head, body = b.split(b"end_header\n")
    lines = head.decode().splitlines()
    assert lines[:3] == ["ply", "format binary_little_endian 1.0", "element vertex 3"]
    assert lines[3] == "property float x" and lines[9] == "property float f_dc_0"
    assert lines[12] == "property float f_rest_0" and lines[56] == "property float f_rest_44"
    assert lines[57:] == ["property float opacity"] + [f"property float scale_{c}" for c in range(3)] + \
        [f"property float rot_{c}" for c in range(4)]
    rec = np.frombuffer(body, dtype="<f4").reshape(n, 62)
    for k in range(n):
        assert list(rec[k, :3]) == [1000 * k + c for c in range(3)] and not rec[k, 3:6].any()
        assert list(rec[k, 6:9]) == [1000 * k + 100 + c for c in range(3)]            # f_dc = sh[0]
        for i in range(45):                                                           # f_rest_i
            assert rec[k, 9 + i] == 1000 * k + 100 + 3 * (1 + i // 3) + i % 3
        assert rec[k, 54] == 1000 * k + 200
        assert list(rec[k, 55:58]) == [1000 * k + 300 + c for c in range(3)]
        assert list(rec[k, 58:62]) == [1000 * k + 400 + c for c in range(4)]
