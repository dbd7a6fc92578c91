"""Shared test setup: the `gpu` marker, repo on sys.path, device fixtures."""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI)")


@pytest.fixture(scope="session")
def dev():
    from ironmill_amd import Device
    d = Device(0)
    yield d


@pytest.fixture(scope="session")
def stream(dev):
    s = dev.stream()
    yield s
    s.sync()


def rel_l2(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


# fp32 accumulate, fp16 out
REL_L2_TOL = 1e-3
MAX_ABS_TOL = 2e-2


def assert_close(got, ref, rel=REL_L2_TOL, max_abs=MAX_ABS_TOL, what="", ulps=1):
    """rel-L2 against the f32/f64 reference, and max-abs on fp16 outputs.

    The reference path's outputs are fp16 too (`half(acc)` in the kernels), so
    the element-wise bound compares `got` with the reference rounded to fp16.
    Where |ref| >= 32 one fp16 step is >= 2^-5 > 2e-2, so two correct fp16
    results one rounding apart would already exceed 2e-2; there the bound is
    `ulps` fp16 steps of the reference value instead:
    max(max_abs, ulps * ulp16(ref)).  Comparisons of the GPU path (fp16 scales
    and zeros, the reference's GPU upload format) with the CPU path (f32 scales)
    use ulps=2: the scale rounding (<= 2^-11 relative) adds up to one step.
    """
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    r = rel_l2(got, ref)
    ref16 = ref.astype(np.float16)
    err = np.abs(got - ref16.astype(np.float64))
    allowed = np.maximum(max_abs, ulps * np.spacing(np.abs(ref16)).astype(np.float64))
    worst = float(np.max(err / allowed)) if got.size else 0.0
    m = float(np.max(err)) if got.size else 0.0
    assert r <= rel and worst <= 1.0, (
        f"{what}: rel_l2={r:.3e} (tol {rel}) max_abs={m:.3e} (bound max({max_abs}, {ulps} ulp16)), "
        f"worst err/bound={worst:.2f}")
    return r, m


# The decoder tests' bound on logits (tests/test_decode_sensitivity.py measures why):
# every stored activation is f16, so sums in another order round some stored values one
# step apart and the layers amplify those steps.  Two oracle variants show how far that
# moves the logits on the test's own inputs: B32, the GPU upload's weight semantics summing
# in f32 instead of f64 (B), and A, the reference's CPU path (weights rounded to f16).  The
# GPU is held to 1e-3 against B, or to twice B32's distance from B, or to A's distance from
# B -- no further from the exact computation than the reference's own CPU path -- and to
# that bound plus A's distance from B against A (the triangle inequality).  Both measured
# distances are held to SPREAD_CAP, so the bound cannot loosen with the data.
SPREAD_CAP = 2e-3


def assert_decoder_logits(got, want_a, want_b, want_b32, what=""):
    """got: GPU logits; A: the reference's CPU path (f16 weights, f32 sums); B / B32: the
    GPU upload's weight semantics summing in f64 / f32.  Returns (rel(GPU,B), rel(GPU,A),
    spread, rel(A,B))."""
    sens = rel_l2(want_b32, want_b)
    ab = rel_l2(want_a, want_b)
    gb, ga = rel_l2(got, want_b), rel_l2(got, want_a)
    print(f"{what}: GPU-B {gb:.2e}  GPU-A {ga:.2e}  | oracle spread B32-B {sens:.2e}  A-B {ab:.2e}", flush=True)
    assert np.all(np.isfinite(np.asarray(got, np.float64))), f"{what}: non-finite logits"
    assert sens <= SPREAD_CAP and ab <= SPREAD_CAP, f"{what}: oracle spreads {sens:.3e} / {ab:.3e} exceed the cap"
    bound = max(1e-3, 2 * sens, ab)
    assert gb <= bound, f"{what}: rel(GPU, B) {gb:.3e} (bound {bound:.3e})"
    assert ga <= bound + ab, f"{what}: rel(GPU, A) {ga:.3e} (bound {bound + ab:.3e})"
    return gb, ga, sens, ab
