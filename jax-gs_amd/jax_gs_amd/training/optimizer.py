"""The reference trainer's optimizer on the GPU: one masked Adam step of the five
Gaussian arrays in one kernel launch.

Mirrors train.py:127-155 (``optax.multi_transform`` of one ``optax.adam`` per array,
the means' learning rate on ``optax.exponential_decay``), trainer.py:44-53
(``_mask_updates``) and ``optax.apply_updates``; the per-element arithmetic runs in
``gs_adam_step``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable, Dict, Union

import numpy as np
import torch

from .. import _lib
from ..core.gaussians import Gaussians
from ..renderer._buffers import as_bytes

FIELDS = ("means", "scales", "quaternions", "opacities", "sh_coeffs")
LearningRate = Union[float, Callable[[int], float]]


def exponential_decay(init_value: float, transition_steps: int, decay_rate: float) -> Callable[[int], float]:
    """optax.exponential_decay (no staircase, transition_begin 0), evaluated in float32."""

    def schedule(count: int) -> float:
        if count <= 0:
            return float(np.float32(init_value))
        p = np.float32(count) / np.float32(transition_steps)
        return float(np.float32(np.float32(init_value) * np.power(np.float32(decay_rate), p)))

    return schedule


@dataclass
class AdamState:
    """First and second moments per array (zeros at init) and the step count."""
    mu: Dict[str, torch.Tensor]
    nu: Dict[str, torch.Tensor]
    count: int = 0


class Adam:
    """optax.adam per parameter array with its own learning rate (a float or a schedule
    of the step count), b1 0.9, b2 0.999, eps 1e-8."""

    def __init__(self, learning_rates: Dict[str, LearningRate], b1: float = 0.9, b2: float = 0.999,
                 eps: float = 1e-8):
        missing = [f for f in FIELDS if f not in learning_rates]
        if missing:
            raise ValueError(f"Adam: no learning rate for {missing}")
        self.lrs = dict(learning_rates)
        self.b1, self.b2, self.eps = float(b1), float(b2), float(eps)

    def init(self, params: Gaussians) -> AdamState:
        return AdamState(mu={f: torch.zeros_like(getattr(params, f)) for f in FIELDS},
                         nu={f: torch.zeros_like(getattr(params, f)) for f in FIELDS}, count=0)

    def lr_at(self, field: str, count: int) -> float:
        lr = self.lrs[field]
        return float(lr(count)) if callable(lr) else float(lr)

    def step(self, params: Gaussians, grads: Gaussians, state: AdamState, active_mask=None) -> AdamState:
        """Update params and the moments in place (trainer.py:70-77): rows whose
        active_mask entry is False keep their parameters; returns the state."""
        n = params.means.shape[0]
        dev = params.means.device
        arrays = []
        for f in FIELDS:
            p, g = getattr(params, f), getattr(grads, f)
            m, v = state.mu[f], state.nu[f]
            for name, t in (("param", p), ("grad", g), ("mu", m), ("nu", v)):
                if t.dtype != torch.float32 or not t.is_contiguous() or t.device != dev or t.shape != p.shape:
                    raise ValueError(f"Adam: {f} {name} must be a contiguous float32 tensor shaped like the "
                                     f"parameter on {dev}")
            arrays.append((p, g, m, v, p.numel(), p.numel() // max(n, 1), self.lr_at(f, state.count)))
        act = None
        if active_mask is not None:
            act = as_bytes(torch.as_tensor(active_mask, device=dev))
            if act.numel() != n:
                raise ValueError(f"Adam: active_mask has {act.numel()} entries for {n} Gaussians")
        k = len(arrays)
        P = ctypes.c_void_p * k
        _lib.call("gs_adam_step", _lib.stream_handle(dev), k, P(*[a[0].data_ptr() for a in arrays]),
                  P(*[a[1].data_ptr() for a in arrays]), P(*[a[2].data_ptr() for a in arrays]),
                  P(*[a[3].data_ptr() for a in arrays]), (ctypes.c_int64 * k)(*[a[4] for a in arrays]),
                  (ctypes.c_int * k)(*[a[5] for a in arrays]), (ctypes.c_double * k)(*[a[6] for a in arrays]),
                  _lib.ptr(act), n, state.count + 1, self.b1, self.b2, self.eps)
        state.count += 1
        return state


def make_optimizer(extent: float, num_iterations: int) -> Adam:
    """train.py:127-155: means 0.00016*extent*3 decaying to 0.0000016*extent*3 over the
    run; scales 0.005, quaternions 0.001, opacities 0.05, SH 0.0025."""
    lr_init = 0.00016 * extent * 3.0
    lr_end = 0.0000016 * extent * 3.0
    return Adam({"means": exponential_decay(lr_init, num_iterations, lr_end / lr_init), "scales": 0.005,
                 "quaternions": 0.001, "opacities": 0.05, "sh_coeffs": 0.0025})
