"""CPU oracle of the tiled Gaussian-splatting rasterizer -- TEST INFRASTRUCTURE ONLY.

This package is the checker the GPU path is compared with.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import it;
the product package (``jax-gs_amd/jax_gs_amd``) never imports, loads or calls it.

It wraps ``libgsoracle.so`` (``gs_oracle.c`` / ``gs_oracle_impl.h``), a C restatement
of the reference ghif/jax-gs in float32 (``dtype=np.float32``) and float64
(``dtype=np.float64``), and restates in NumPy the host-side glue of
``jax_gs/renderer/renderer.py:15-107`` (view-independent plumbing, tile ranges and
the ``extras`` dict) and the losses of ``jax_gs/training/losses.py:4-75`` (L1, MSE,
SSIM with its VJP written out by hand).

Pinning (what checks this oracle independently of its own formulas) is listed in
``tests/test_oracle.py``; every function below is pinned there.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBPATH = os.path.join(_HERE, "libgsoracle.so")
_lib = None

TILE_SIZE = 16
BLOCK_SIZE = 512
MAX_TILE_INTERACTIONS = 4096


def build(force: bool = False) -> str:
    """Compile libgsoracle.so with the committed Makefile (gcc only)."""
    if force or not os.path.exists(_LIBPATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []) + ["libgsoracle.so"], check=True)
    return _LIBPATH


def lib():
    global _lib
    if _lib is None:
        build()
        _lib = ctypes.CDLL(_LIBPATH)
        _lib.gso_expf.restype = ctypes.c_float
        _lib.gso_expf.argtypes = [ctypes.c_float]
        _lib.gso_set_threads.argtypes = [ctypes.c_int]
    return _lib


def set_threads(n: int) -> None:
    """Threads of the oracle's parallel loops (OpenMP; default: OMP_NUM_THREADS or all CPUs)."""
    lib().gso_set_threads(int(n))


def threads() -> int:
    return int(lib().gso_max_threads())


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _sfx(dtype):
    return "f" if np.dtype(dtype) == np.float32 else "d"


def _real(dtype):
    return ctypes.c_float if np.dtype(dtype) == np.float32 else ctypes.c_double


def expf(x: float) -> float:
    """The float32 exp of the restatement (and of the product's preprocess kernel)."""
    return float(lib().gso_expf(ctypes.c_float(x)))


def preprocess(means, scales, quats, sh, w2c, W, H, fx, fy, cx, cy, sh_degree, mask=None, dtype=np.float32):
    """projection.py:6-79 + gaussians.py:58-92 + renderer.py:40-49 + sh.py:25-74."""
    L = lib()
    means, scales, quats, sh, w2c = (_c(a, dtype) for a in (means, scales, quats, sh, w2c))
    n = means.shape[0]
    K = sh.shape[1]
    out = dict(
        means2d=np.zeros((n, 2), dtype), cov2d=np.zeros((n, 2, 2), dtype), radii=np.zeros((n,), dtype),
        valid=np.zeros((n,), np.uint8), depths=np.zeros((n,), dtype), colors=np.zeros((n, 3), dtype))
    m = None if mask is None else _c(mask, np.uint8)
    R = _real(dtype)
    fn = getattr(L, "gso_preprocess_" + _sfx(dtype))
    rc = fn(ctypes.c_int64(n), ctypes.c_int(K), ctypes.c_int(sh_degree), _p(means), _p(scales), _p(quats), None,
            _p(sh), _p(m), _p(w2c.reshape(16)), ctypes.c_int(W), ctypes.c_int(H), R(fx), R(fy), R(cx), R(cy),
            _p(out["means2d"]), _p(out["cov2d"]), _p(out["radii"]), _p(out["valid"]), _p(out["depths"]),
            _p(out["colors"]))
    assert rc == 0
    out["valid"] = out["valid"].astype(bool)
    return out


def tile_interactions(means2d, radii, valid, depths, H, W, dtype=np.float32):
    """rasterizer.py:12-116: (sorted_tile_ids[L], sorted_gaussian_ids[L], n_interactions)."""
    means2d, radii, depths = (_c(a, dtype) for a in (means2d, radii, depths))
    v = _c(valid, np.uint8)
    n = means2d.shape[0]
    Lsz = max(256 * n, BLOCK_SIZE)
    st = np.empty((Lsz,), np.int32)  # every slot is written
    sg = np.empty((Lsz,), np.int32)
    cnt = ctypes.c_int64(0)
    fn = getattr(lib(), "gso_tile_interactions_" + _sfx(dtype))
    rc = fn(ctypes.c_int64(n), _p(means2d), _p(radii), _p(v), _p(depths), ctypes.c_int(W), ctypes.c_int(H),
            _p(st), _p(sg), ctypes.byref(cnt))
    if rc != 0:
        raise MemoryError("oracle tile_interactions could not allocate its slot arrays")
    return st, sg, int(cnt.value)


def render_tiles(means2d, cov2d, opacities, colors, sorted_tiles, sorted_gids, H, W, background=None,
                 tpu_gather=False, dtype=np.float32):
    """rasterizer.py:119-248 (or rasterizer_tpu.py:13-135 with tpu_gather=True).

    Returns (image[H,W,3], final_T[H,W], n_contrib[H,W])."""
    means2d, cov2d, opacities, colors = (_c(a, dtype) for a in (means2d, cov2d, opacities, colors))
    bg = _c(np.zeros(3) if background is None else background, dtype)
    st, sg = _c(sorted_tiles, np.int32), _c(sorted_gids, np.int32)
    img = np.zeros((H, W, 3), dtype)
    fT = np.zeros((H, W), dtype)
    nc = np.zeros((H, W), np.int32)
    fn = getattr(lib(), "gso_render_tiles_" + _sfx(dtype))
    rc = fn(ctypes.c_int64(means2d.shape[0]), _p(means2d), _p(cov2d), _p(opacities), _p(colors), _p(st), _p(sg),
            ctypes.c_int64(st.shape[0]), ctypes.c_int(W), ctypes.c_int(H), _p(bg), ctypes.c_int(int(tpu_gather)),
            _p(img), _p(fT), _p(nc))
    assert rc == 0
    return img, fT, nc


def render_tiles_bwd(means2d, cov2d, opacities, colors, sorted_tiles, sorted_gids, H, W, g_image, background=None,
                     tpu_gather=False, dtype=np.float32):
    """Reverse-mode derivative of render_tiles: cotangents of (means2d, cov2d, opacity logits, colors, bg)."""
    means2d, cov2d, opacities, colors, g_image = (_c(a, dtype) for a in (means2d, cov2d, opacities, colors, g_image))
    bg = _c(np.zeros(3) if background is None else background, dtype)
    st, sg = _c(sorted_tiles, np.int32), _c(sorted_gids, np.int32)
    n = means2d.shape[0]
    out = dict(means2d=np.zeros((n, 2), dtype), cov2d=np.zeros((n, 2, 2), dtype), opacities=np.zeros((n, 1), dtype),
               colors=np.zeros((n, 3), dtype), background=np.zeros((3,), dtype))
    fn = getattr(lib(), "gso_render_tiles_bwd_" + _sfx(dtype))
    rc = fn(ctypes.c_int64(n), _p(means2d), _p(cov2d), _p(opacities), _p(colors), _p(st), _p(sg),
            ctypes.c_int64(st.shape[0]), ctypes.c_int(W), ctypes.c_int(H), _p(bg), ctypes.c_int(int(tpu_gather)),
            _p(g_image), _p(out["means2d"]), _p(out["cov2d"]), _p(out["opacities"]), _p(out["colors"]),
            _p(out["background"]))
    if rc != 0:
        raise MemoryError("oracle render_tiles_bwd could not allocate")
    return out


def preprocess_bwd(means, scales, quats, sh, w2c, fx, fy, sh_degree, g_means2d, g_cov2d, g_colors, dtype=np.float32):
    """Reverse-mode derivative of preprocess w.r.t. means, scales, quaternions, sh_coeffs
    and the camera's W2C (key "W2C", [4,4], row 3 zero)."""
    means, scales, quats, sh, w2c, g_means2d, g_cov2d, g_colors = (
        _c(a, dtype) for a in (means, scales, quats, sh, w2c, g_means2d, g_cov2d, g_colors))
    n, K = means.shape[0], sh.shape[1]
    out = dict(means=np.zeros((n, 3), dtype), scales=np.zeros((n, 3), dtype), quaternions=np.zeros((n, 4), dtype),
               sh_coeffs=np.zeros((n, K, 3), dtype), W2C=np.zeros((4, 4), dtype))
    R = _real(dtype)
    fn = getattr(lib(), "gso_preprocess_bwd_w2c_" + _sfx(dtype))
    rc = fn(ctypes.c_int64(n), ctypes.c_int(K), ctypes.c_int(sh_degree), _p(means), _p(scales), _p(quats), _p(sh),
            _p(w2c.reshape(16)), R(fx), R(fy), _p(g_means2d), _p(g_cov2d), _p(g_colors), _p(out["means"]),
            _p(out["scales"]), _p(out["quaternions"]), _p(out["sh_coeffs"]), _p(out["W2C"]))
    assert rc == 0
    return out


def eval_sh(sh_degree, sh_coeffs, view_dirs, dtype=np.float32):
    """sh.py:25-74: the SH expansion [N, 3] (no +0.5, no clip)."""
    sh, d = _c(sh_coeffs, dtype), _c(view_dirs, dtype)
    n, K = sh.shape[0], sh.shape[1]
    out = np.zeros((n, 3), dtype)
    rc = getattr(lib(), "gso_eval_sh_" + _sfx(dtype))(ctypes.c_int64(n), ctypes.c_int(K), ctypes.c_int(sh_degree),
                                                        _p(sh), _p(d), _p(out))
    assert rc == 0
    return out


def eval_sh_vjp(sh_degree, sh_coeffs, view_dirs, g_colors, dtype=np.float32):
    """Cotangents (sh_coeffs [N, K, 3], view_dirs [N, 3]) of eval_sh for g_colors [N, 3]."""
    sh, d, g = _c(sh_coeffs, dtype), _c(view_dirs, dtype), _c(g_colors, dtype)
    n, K = sh.shape[0], sh.shape[1]
    g_sh = np.zeros((n, K, 3), dtype)
    g_d = np.zeros((n, 3), dtype)
    rc = getattr(lib(), "gso_eval_sh_bwd_" + _sfx(dtype))(ctypes.c_int64(n), ctypes.c_int(K),
                                                            ctypes.c_int(sh_degree), _p(sh), _p(d), _p(g), _p(g_sh),
                                                            _p(g_d))
    assert rc == 0
    return g_sh, g_d


def tile_boundaries(sorted_tiles, num_tiles):
    """renderer.py:60: jnp.searchsorted(sorted_tile_ids, arange(T+1)) (side='left')."""
    st = np.asarray(sorted_tiles)
    return np.searchsorted(st, np.arange(num_tiles + 1, dtype=st.dtype), side="left").astype(np.int32)


def extras_from(pre, sorted_tiles, n_interactions, H, W):
    """renderer.py:57-90 restated in NumPy (int32/float32 like the reference)."""
    TX, TY = (W + 15) // 16, (H + 15) // 16
    T = TX * TY
    b = tile_boundaries(sorted_tiles, T)
    counts = (b[1:] - b[:-1]).astype(np.int32)
    m2, r = pre["means2d"], pre["radii"]
    f = m2.dtype.type
    minx = np.clip(m2[:, 0] - r, f(0), f(W - 1))
    maxx = np.clip(m2[:, 0] + r, f(0), f(W - 1))
    miny = np.clip(m2[:, 1] - r, f(0), f(H - 1))
    maxy = np.clip(m2[:, 1] + r, f(0), f(H - 1))
    with np.errstate(invalid="ignore"):
        tminx = np.nan_to_num(np.floor(minx / f(16))).astype(np.int32)
        tmaxx = np.nan_to_num(np.floor(maxx / f(16))).astype(np.int32)
        tminy = np.nan_to_num(np.floor(miny / f(16))).astype(np.int32)
        tmaxy = np.nan_to_num(np.floor(maxy / f(16))).astype(np.int32)
        on = (m2[:, 0] + r > 0) & (m2[:, 0] - r < W) & (m2[:, 1] + r > 0) & (m2[:, 1] - r < H)
    capped = ((tmaxx - tminx + 1) > 16) | ((tmaxy - tminy + 1) > 16)
    return dict(
        radii=r, valid_mask=pre["valid"], n_interactions=np.int32(n_interactions),
        mean_interactions_per_tile=np.float32(n_interactions) / np.float32(max(T, 1)),
        max_interactions_per_tile=np.int32(counts.max()) if T > 0 else np.int32(0),
        overflow_tiles=np.int32((counts > BLOCK_SIZE).sum()),
        overflow_interactions=np.int32(np.maximum(counts - BLOCK_SIZE, 0).sum()),
        truncated_tiles=np.int32((counts > MAX_TILE_INTERACTIONS).sum()),
        truncated_interactions=np.int32(np.maximum(counts - MAX_TILE_INTERACTIONS, 0).sum()),
        radius_cap_violations=np.int32((capped & pre["valid"] & on).sum()),
        tile_boundaries=b)


def render(params, cam, background=None, mask=None, sh_degree=0, tpu_gather=False, dtype=np.float32):
    """renderer.py:15-107 restated: returns (image, extras, residuals-for-backward).

    params: dict with means, scales, quaternions, opacities, sh_coeffs (NumPy).
    cam: dict with W, H, fx, fy, cx, cy (Python numbers) and W2C (4x4)."""
    f = np.dtype(dtype).type
    W, H = cam["W"], cam["H"]
    args = (f(cam["fx"]), f(cam["fy"]), f(cam["cx"]), f(cam["cy"]))
    pre = preprocess(params["means"], params["scales"], params["quaternions"], params["sh_coeffs"], cam["W2C"], W, H,
                     *args, sh_degree, mask=mask, dtype=dtype)
    st, sg, n = tile_interactions(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W, dtype=dtype)
    bg = np.zeros(3, dtype) if background is None else np.asarray(background, dtype)
    img, fT, nc = render_tiles(pre["means2d"], pre["cov2d"], params["opacities"], pre["colors"], st, sg, H, W, bg,
                               tpu_gather=tpu_gather, dtype=dtype)
    extras = extras_from(pre, st, n, H, W)
    res = dict(pre=pre, sorted_tiles=st, sorted_gids=sg, background=bg, final_T=fT, n_contrib=nc)
    return img, extras, res


def render_vjp(params, cam, res, g_image, sh_degree=0, tpu_gather=False, dtype=np.float32):
    """Cotangents of the five Gaussian arrays (and background) for an image cotangent."""
    f = np.dtype(dtype).type
    pre = res["pre"]
    gt = render_tiles_bwd(pre["means2d"], pre["cov2d"], params["opacities"], pre["colors"], res["sorted_tiles"],
                          res["sorted_gids"], cam["H"], cam["W"], g_image, res["background"], tpu_gather=tpu_gather,
                          dtype=dtype)
    gp = preprocess_bwd(params["means"], params["scales"], params["quaternions"], params["sh_coeffs"], cam["W2C"],
                        f(cam["fx"]), f(cam["fy"]), sh_degree, gt["means2d"], gt["cov2d"], gt["colors"], dtype=dtype)
    return dict(means=gp["means"], scales=gp["scales"], quaternions=gp["quaternions"], opacities=gt["opacities"],
                sh_coeffs=gp["sh_coeffs"], background=gt["background"], W2C=gp["W2C"])


def densify(g_means, means, w2c, fx, fy, W, H, valid, radii, grad_accum, denom, max_radii, active=None,
            dtype=np.float32):
    """trainer.py:143-159: returns updated (grad_accum, denom, max_radii) (inputs untouched).

    focal = (fx + fy) / 2 and the scale W*H*3 enter as the float32 scalars JAX's weak
    typing makes of the Python floats."""
    f = np.dtype(dtype).type
    g_means, means, w2c, radii = (_c(a, dtype) for a in (g_means, means, w2c, radii))
    ga = _c(grad_accum, dtype).copy()
    de = _c(denom, np.int32).copy()
    mr = _c(max_radii, dtype).copy()
    v = _c(valid, np.uint8)
    a = None if active is None else _c(active, np.uint8)
    fn = getattr(lib(), "gso_densify_" + _sfx(dtype))
    R = _real(dtype)
    rc = fn(ctypes.c_int64(means.shape[0]), _p(g_means), _p(means), _p(w2c.reshape(16)), R(f((fx + fy) / 2.0)),
            R(f(float(W) * float(H) * 3.0)), _p(v), _p(a), _p(radii), _p(ga), _p(de), _p(mr))
    assert rc == 0
    return ga, de, mr


def l1_loss_and_grad(image, target):
    """losses.py:4-8: mean(|pred - target|) and its seed sign(d) * (1/count)."""
    d = image.astype(np.float32) - target.astype(np.float32)
    cnt = np.float32(d.size)
    return np.float32(np.abs(d).astype(np.float64).mean()), (np.sign(d) * (np.float32(1) / cnt)).astype(np.float32)


def mse_loss_and_grad(image, target):
    """losses.py:10-14: mean((pred - target)^2) and its seed 2 d * (1/count)."""
    d = image.astype(np.float32) - target.astype(np.float32)
    cnt = np.float32(d.size)
    return np.float32((d.astype(np.float64) ** 2).mean()), (np.float32(2) * d * (np.float32(1) / cnt)).astype(np.float32)


# ---------------------------------------------------------------------------------------
# SSIM (losses.py:16-75): separable Gaussian window, 'SAME' zero padding, clipped map.
SSIM_C1 = 0.01 ** 2
SSIM_C2 = 0.03 ** 2


def ssim_window(size=11, sigma=1.5, dtype=np.float32):
    """losses.py:24-29: taps exp(-x^2 / (2 sigma^2)) for x = -(size//2)..size//2, normalised."""
    x = (np.arange(size) - size // 2).astype(dtype)
    k = np.exp(-(x * x) / dtype(2.0 * sigma * sigma)).astype(dtype)
    return (k / k.sum(dtype=dtype)).astype(dtype)


def ssim_blur(img, w, adjoint=False):
    """losses.py:35-47: depthwise correlation with w along H, then along W, each with
    XLA's 'SAME' zero padding: (L-1)//2 before and L//2 after for L = len(w) taps, so
    output i reads input i + k - (L-1)//2.  img is [H, W, C].  adjoint=True applies the
    transposed operator (the correlation with the reversed taps and swapped padding; for
    odd L, the same blur)."""
    H, W = img.shape[:2]
    L = len(w)
    lo = (L - 1) // 2
    if adjoint:
        w = w[::-1]
        lo = L - 1 - lo
    hi = L - 1 - lo
    dt = img.dtype
    p = np.zeros((H + L - 1,) + img.shape[1:], dt)
    p[lo:lo + H] = img
    v = np.zeros_like(img)
    for k in range(L):
        v = v + w[k] * p[k:k + H]
    p = np.zeros((H, W + L - 1) + img.shape[2:], dt)
    p[:, lo:lo + W] = v
    out = np.zeros_like(img)
    for k in range(L):
        out = out + w[k] * p[:, k:k + W]
    del hi
    return out


def _ssim_parts(img1, img2, dtype, window_size=11):
    w = ssim_window(window_size, dtype=dtype)
    x = np.asarray(img1, dtype)
    y = np.asarray(img2, dtype)
    mu1, mu2 = ssim_blur(x, w), ssim_blur(y, w)
    m11, m22, m12 = mu1 * mu1, mu2 * mu2, mu1 * mu2
    d11 = ssim_blur(x * x, w) - m11
    d22 = ssim_blur(y * y, w) - m22
    s11, s22 = np.maximum(dtype(0), d11), np.maximum(dtype(0), d22)
    s12 = ssim_blur(x * y, w) - m12
    c1, c2 = dtype(SSIM_C1), dtype(SSIM_C2)
    A, B = dtype(2) * m12 + c1, dtype(2) * s12 + c2
    Cc, D = m11 + m22 + c1, s11 + s22 + c2
    raw = (A * B) / (Cc * D)
    return dict(w=w, x=x, y=y, mu1=mu1, mu2=mu2, d11=d11, A=A, B=B, Cc=Cc, D=D, raw=raw)


def ssim_map(img1, img2, dtype=np.float64, window_size=11):
    """losses.py:49-64: the clipped per-value SSIM map [H, W, C]."""
    return np.clip(_ssim_parts(img1, img2, dtype, window_size)["raw"], -1.0, 1.0)


def ssim(img1, img2, dtype=np.float64, window_size=11):
    """losses.py:16-68 (size_average): mean of the clipped SSIM map."""
    return ssim_map(img1, img2, dtype, window_size).astype(np.float64).mean()


def d_ssim_loss(pred, target, dtype=np.float64):
    """losses.py:70-75: max(0, (1 - ssim) / 2)."""
    return max(0.0, (1.0 - ssim(pred, target, dtype)) / 2.0)


def _tie_grad(z):
    """d max(0, z)/dz with JAX's balanced tie: 1 above, 1/2 at 0, 0 below."""
    return np.where(z > 0, 1.0, np.where(z == 0, 0.5, 0.0))


def ssim_vjp(img1, img2, g_ssim, dtype=np.float64, window_size=11):
    """Cotangent of img1 for the mean SSIM given its cotangent g_ssim: reverse-mode AD
    of losses.py:49-68 written out by hand.  Ties of max/clip pass half the cotangent
    (lax.max/min).  The blur's adjoint is ssim_blur(..., adjoint=True)."""
    P = _ssim_parts(img1, img2, dtype, window_size)
    raw, A, B, Cc, D = P["raw"], P["A"], P["B"], P["Cc"], P["D"]
    # clip(raw, -1, 1) = minimum(1, maximum(-1, raw))
    clip_d = _tie_grad(raw + 1.0) * _tie_grad(1.0 - raw)
    G = dtype(g_ssim) / dtype(raw.size) * clip_d.astype(dtype)
    num, den = A * B, Cc * D
    dnum, dden = G / den, -G * num / (den * den)
    dA, dB, dCc, dD = dnum * B, dnum * A, dden * D, dden * Cc
    de12 = dtype(2) * dB                                   # s12 = e12 - m12
    dm12 = dtype(2) * dA - de12
    de11 = dD * _tie_grad(P["d11"]).astype(dtype)          # s11 = max(0, e11 - m11)
    dm11 = dCc - de11
    dmu1 = dtype(2) * P["mu1"] * dm11 + P["mu2"] * dm12    # m11 = mu1^2, m12 = mu1 mu2
    w = P["w"]
    return (ssim_blur(dmu1, w, True) + dtype(2) * P["x"] * ssim_blur(de11, w, True)
            + P["y"] * ssim_blur(de12, w, True))


def d_ssim_vjp(pred, target, g, dtype=np.float64):
    """Cotangent of pred for d_ssim_loss = max(0, (1 - ssim) / 2) with cotangent g."""
    s = ssim(pred, target, dtype)
    return ssim_vjp(pred, target, -0.5 * g * float(_tie_grad(np.float64((1.0 - s) / 2.0))), dtype)


# ---------------------------------------------------------------------------------------
# Optimizer (train.py:127-155 optax.multi_transform of optax.adam; trainer.py:44-53
# _mask_updates; optax.apply_updates), restated operation by operation in float32.
def exponential_decay(init_value, transition_steps, decay_rate):
    """optax.exponential_decay (transition_begin 0, no staircase): init * rate^(count/steps)."""
    def schedule(count):
        if count <= 0:
            return np.float32(init_value)
        p = np.float32(count) / np.float32(transition_steps)
        return np.float32(np.float32(init_value) * np.power(np.float32(decay_rate), p))
    return schedule


def adam_step(param, grad, mu, nu, count, lr, active=None, b1=0.9, b2=0.999, eps=1e-8):
    """One optax.adam update of one parameter array followed by the trainer's row mask
    and optax.apply_updates.  count is the optimizer's step count before this update
    (the learning-rate schedule is evaluated at it); returns (param, mu, nu) new."""
    f = np.float32
    g = grad.astype(f)
    mu = (f(1.0 - b1) * g + f(b1) * mu).astype(f)                  # update_moment
    nu = (f(1.0 - b2) * (g * g) + f(b2) * nu).astype(f)            # update_moment_per_elem_norm
    t = count + 1
    bc1 = f(1.0) - np.power(f(b1), f(t))                            # bias_correction
    bc2 = f(1.0) - np.power(f(b2), f(t))
    u = (mu / bc1) / (np.sqrt(nu / bc2) + f(eps))                   # eps_root = 0
    u = u * f(-lr)                                                  # scale_by_learning_rate
    if active is not None:                                          # _mask_updates
        m = np.asarray(active, bool).reshape((-1,) + (1,) * (param.ndim - 1))
        u = np.where(m, u, f(0.0))
    return (param + u).astype(f), mu, nu


def expf_array(a):
    """gso_expf elementwise (float32)."""
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty_like(a)
    lib().gso_expf_array(ctypes.c_int64(a.size), _p(a), _p(out))
    return out


# ---------------------------------------------------------------------------------------
# Densification (density.py:98-211 densify_and_prune, :63-67 _reset_accumulators)
def densify_and_prune(state, noise, densify_enabled=True, grad_threshold=0.0002, min_opacity=0.005, extent=5.0,
                      max_screen_size=512):
    """Restates densify_and_prune on NumPy copies.  state: dict with the five parameter
    arrays (means, scales, quaternions, opacities, sh_coeffs), 'moments' (dict of extra
    arrays with the capacity as leading dimension, gathered like the parameters), 'active'
    (bool [M]), 'grad_accum', 'denom', 'max_radii'.  noise: [M, 3] standard normal draws
    (the reference draws them with jax.random.normal).  Returns the new state and a dict
    of counts."""
    f = np.float32
    M = state["active"].shape[0]
    active = state["active"].astype(bool)
    sig = f(1.0) / (f(1.0) + expf_array(-state["opacities"][:, 0]))
    prune = sig < f(min_opacity)
    max_scales = expf_array(state["scales"]).max(axis=-1)
    prune |= max_scales > f(0.1 * extent)
    prune |= state["max_radii"] > f(max_screen_size)
    prune &= active
    after = active & ~prune
    denom = state["denom"]
    with np.errstate(divide="ignore", invalid="ignore"):
        avg = np.where(denom > 0, state["grad_accum"] / denom.astype(f), f(0.0)).astype(f)
    densify = (avg >= f(grad_threshold)) & after
    split = densify & (max_scales > f(0.01 * extent))
    clone = densify & ~split
    empty = ~after
    can = bool(clone.sum() + split.sum() <= empty.sum()) and bool(densify_enabled)
    if not can:
        clone[:] = False
        split[:] = False
    nc, ns = int(clone.sum()), int(split.sum())
    # stable argsorts of (not empty), (not clone), (not split): the k-th empty slot takes the
    # k-th clone source, then the (k - nc)-th split source
    empty_idx = np.argsort((~empty).astype(np.int8), kind="stable")
    clone_src = np.argsort((~clone).astype(np.int8), kind="stable")
    split_src = np.argsort((~split).astype(np.int8), kind="stable")
    gather = np.arange(M)
    is_split_dest = np.zeros(M, bool)
    for k in range(nc + ns):
        dst = empty_idx[k]
        gather[dst] = clone_src[k] if k < nc else split_src[k - nc]
        is_split_dest[dst] = k >= nc
    out = {}
    for key in ("means", "scales", "quaternions", "opacities", "sh_coeffs"):
        out[key] = state[key][gather].copy()
    out["moments"] = {k: v[gather].copy() for k, v in state.get("moments", {}).items()}
    do_split = split | is_split_dest
    out["scales"] = np.where(do_split[:, None], out["scales"] - f(np.log(1.6)), out["scales"]).astype(f)
    jitter = (noise.astype(f) * expf_array(out["scales"])).astype(f)
    out["means"] = np.where(do_split[:, None], out["means"] + jitter, out["means"]).astype(f)
    added = np.zeros(M, bool)
    added[empty_idx[:nc + ns]] = True
    out["active"] = after | added
    out["grad_accum"] = np.zeros_like(state["grad_accum"])
    out["denom"] = np.zeros_like(state["denom"])
    out["max_radii"] = state["max_radii"].copy()
    return out, dict(clones=nc, splits=ns, pruned=int(prune.sum()), available=int(empty.sum()), gather=gather)


# ---------------------------------------------------------------------------------------
# PLY checkpoint bytes (ply.py:6-123), restated with the reference's structured dtype
def ply_dtype():
    names = (["x", "y", "z", "nx", "ny", "nz", "f_dc_0", "f_dc_1", "f_dc_2"] + [f"f_rest_{i}" for i in range(45)] +
             ["opacity", "scale_0", "scale_1", "scale_2", "rot_0", "rot_1", "rot_2", "rot_3"])
    return [(n, "<f4") for n in names]


def ply_bytes(means, scales, quats, opacities, sh):
    """The file save_ply writes for these arrays (sh [N, 16, 3])."""
    dt = ply_dtype()
    n = means.shape[0]
    data = np.zeros(n, dtype=dt)
    data["x"], data["y"], data["z"] = means[:, 0], means[:, 1], means[:, 2]
    f_dc = sh[:, 0, :].reshape(-1, 3)
    f_rest = sh[:, 1:, :].reshape(-1, 45)
    for c in range(3):
        data[f"f_dc_{c}"] = f_dc[:, c]
    for i in range(45):
        data[f"f_rest_{i}"] = f_rest[:, i]
    data["opacity"] = opacities[:, 0]
    for c in range(3):
        data[f"scale_{c}"] = scales[:, c]
    for c in range(4):
        data[f"rot_{c}"] = quats[:, c]
    head = b"ply\nformat binary_little_endian 1.0\n" + f"element vertex {n}\n".encode()
    head += b"".join(f"property float {name}\n".encode() for name, _ in dt) + b"end_header\n"
    return head + data.tobytes()
