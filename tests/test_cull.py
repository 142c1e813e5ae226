"""The compositing kernels' entry cull never drops an entry a pixel could blend.

gs::entry_misses_rect (jax-gs_amd/csrc/gs_cull.h, shared with the kernels) is compiled
for the host with the kernels' own floating-point settings and fuzzed near the gate's
decision boundary (tests/cull_fuzz.cpp): for every dropped (entry, rectangle) pair, every
pixel centre of the rectangle must fail power > -10 as the kernels compute it.
"""
import os
import shutil
import subprocess

import pytest

_HERE = os.path.dirname(os.path.abspath(__file__))
_CSRC = os.path.join(os.path.dirname(_HERE), "jax-gs_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def fuzz_bin(tmp_path_factory):
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc not found")
    out = str(tmp_path_factory.mktemp("cull") / "cull_fuzz")
    # host-only build; -ffp-contract=off as for the kernels (no contraction beyond the
    # explicit fmaf calls)
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-ffp-contract=off", "-I", _CSRC,
                    os.path.join(_HERE, "cull_fuzz.cpp"), "-o", out], check=True, capture_output=True)
    return out


@pytest.mark.parametrize("seed", [1, 2])
def test_no_false_drop_near_the_gate_boundary(fuzz_bin, seed):
    res = subprocess.run([fuzz_bin, "5000000", str(seed)], capture_output=True, text=True)
    cases, dropped, false_drops, min_margin = res.stdout.split()
    assert int(false_drops) == 0 and res.returncode == 0
    # the fuzz is not vacuous: a large share of the near-boundary cases is dropped, and the
    # closest dropped pixel sits just past the gate
    assert int(dropped) > int(cases) // 10
    assert 0.0 <= float(min_margin) < 0.5


@pytest.fixture(scope="module")
def cap_fuzz_bin(tmp_path_factory):
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc not found")
    out = str(tmp_path_factory.mktemp("cap") / "cap_fuzz")
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-ffp-contract=off", "-I", _CSRC,
                    os.path.join(_HERE, "cap_fuzz.cpp"), "-o", out], check=True, capture_output=True)
    return out


def _cap_fuzz(binary, cases, seed, rule, regime):
    res = subprocess.run([binary, str(cases), str(seed), rule, regime], capture_output=True, text=True)
    n, flagged, violations, margin = res.stdout.split()
    return int(n), int(flagged), int(violations), float(margin), res.returncode


@pytest.mark.parametrize("seed", [1, 2])
def test_cap_flag_holds_for_thin_large_gaussians(cap_fuzz_bin, seed):
    """gs::record_cannot_cap (slot 11 of a compositing record) is set only when no gated pixel
    reaches exp2(q) >= 0.99 as the kernels round q: long thin Gaussians near the cap."""
    n, flagged, violations, margin, rc = _cap_fuzz(cap_fuzz_bin, 200000, seed, "new", "needle")
    assert violations == 0 and rc == 0
    assert flagged > 0 and margin > 0.0


def test_cap_flag_is_set_for_ordinary_gaussians(cap_fuzz_bin):
    """The flag is not vacuous: ordinary Gaussians (eigenvalues 0.3..1e3 px^2, opacity below
    0.98) are flagged, so the backward skips its cap test for practically all of them."""
    n, flagged, violations, margin, rc = _cap_fuzz(cap_fuzz_bin, 200000, 3, "new", "typical")
    assert violations == 0 and rc == 0
    assert flagged >= 0.999 * n


def test_cap_fuzz_finds_the_rounding_blind_rule(cap_fuzz_bin):
    """The fuzz has the power to see a wrong flag: the rule 'op < 0.98 and cov2D positive
    definite', which ignores the rounding of q, is flagged safe for needles whose gated pixels
    reach q well above log2(0.99)."""
    n, flagged, violations, margin, rc = _cap_fuzz(cap_fuzz_bin, 200000, 1, "old", "needle")
    assert violations > 0 and rc != 0 and margin < 0.0
