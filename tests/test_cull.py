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
