"""GPU parity of the bf16 / fp8-e4m3 prefill GEMM (imh_affine_gemm_int4).

Two references, on the same seeded weights W ~ N(0, 0.02) (INT4 group 128) and
activations X ~ N(0, 1) given as bf16:

* the kernel's own arithmetic, restated exactly: a = x / awq rounded once to
  the operand type (oracle.bf16_round / oracle.e4m3_round, pinned against
  torch in test_oracle.py) times the exact weights (q - z16) * s16, summed in
  float64.  The GPU keeps every weight exact and sums in f32, so its bf16
  output must be that value rounded to bf16, up to the f32 sums: within one
  bf16 step plus 2^-18 of the magnitudes those sums carry, sum_k |a| (|q| +
  |z|) s -- the matrix cores form sum a q and the zero-point correction z sum
  a as separate f32 sums, each ~10x sum_k |a (q - z) s| on these weights, so
  on an output near zero their rounding is what remains (the bf16 path's
  codes also carry an offset of 128, which its MFMAs absorb).  Measured on
  1093 x 8036 x 1024 with AWQ: worst 0.49 of this bound at bf16 and fp8.
* the reference's CPU path (dequantize to f16 with f32 scales, f32 matvec,
  oracle.matvec_f16w).  bf16 output rounding alone is ~1.1e-3 relative (8
  significant bits), so the bf16 variant is held to rel-L2 <= 3e-3 there; the
  fp8 variant rounds a to 3 significant bits (~2.5 % relative per element)
  and is held to rel-L2 <= 5e-2 against the CPU path and the bf16 result.
"""
import numpy as np
import pytest

import oracle as O
from conftest import rel_l2
from ironmill_amd import ops, quant

pytestmark = pytest.mark.gpu


def problem(m, n, k, seed, awq):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    s = rng.uniform(0.5, 2.0, k).astype(np.float32) if awq else None
    x = rng.standard_normal((m, k)).astype(np.float32)
    return quant.quantize_int4(w, awq_scales=s), O.bf16_round(x)


def operand(xb, q, prec):
    a = O.bf16_to_f32(xb)
    if q.awq is not None:
        a = (a / q.awq.astype(np.float32)).astype(np.float32)
    return O.bf16_to_f32(O.bf16_round(a)) if prec == ops.GEMM_BF16 else O.e4m3_round(a)


def exact_weights(q):
    codes = O.unpack_int4(q.data.reshape(-1), q.n * q.k).reshape(q.n, q.k // 128, 128).astype(np.float64)
    z = q.zeros.astype(np.float64)[:, :, None]
    s = q.scales.astype(np.float64)[:, :, None]
    return ((codes - z) * s).reshape(q.n, q.k)


def run(dev, stream, q, xb, prec):
    m = xb.shape[0]
    wt = ops.AffineQuantizedWeight(dev, q)
    y = dev.empty((m, q.n), np.uint16)
    ops.encode_affine_gemm_int4(stream, dev.upload(xb), m, wt, y, prec)
    stream.sync()
    return O.bf16_to_f32(y.read())


def weight_magnitudes(q):
    """(|q| + |z|) * s per weight: what the kernel's f32 sums carry per unit of |a|."""
    codes = O.unpack_int4(q.data.reshape(-1), q.n * q.k).reshape(q.n, q.k // 128, 128).astype(np.float64)
    z = np.abs(q.zeros.astype(np.float64))[:, :, None]
    s = np.abs(q.scales.astype(np.float64))[:, :, None]
    return ((codes + z) * s).reshape(q.n, q.k)


def assert_bf16_rounding_of(got, exact, terms, what):
    """got (bf16 values as f32) within one bf16 step of the exact f64 result, plus 2^-18 of
    the magnitudes the f32 sums carry (terms = sum_k |a| (|q| + |z|) s)."""
    mag = np.maximum(np.abs(exact), 1e-30)
    ulp = np.exp2(np.floor(np.log2(mag)) - 7)
    err = np.abs(got.astype(np.float64) - exact)
    worst = float(np.max(err / (ulp + 2.0 ** -18 * terms)))
    assert worst <= 1.0, f"{what}: worst error {worst:.2f} x (bf16 step + 2^-18 sum |a| (|q| + |z|) s)"


def check_exact(got, a, q, what):
    exact = a.astype(np.float64) @ exact_weights(q).T
    terms = np.abs(a).astype(np.float64) @ weight_magnitudes(q).T
    assert_bf16_rounding_of(got, exact, terms, what)


@pytest.mark.parametrize("prec", [ops.GEMM_BF16, ops.GEMM_FP8_E4M3], ids=["bf16", "fp8"])
@pytest.mark.parametrize("m,n,k,awq", [
    (64, 256, 256, False),     # one workgroup tile, split K
    (100, 1000, 1024, True),   # ragged M and N, AWQ
    (33, 2560, 9728, True),    # Qwen3-4B down shape, few tokens: split K
    (1093, 8036, 1024, True),  # 18 x 32 tiles: one round whole, the rest (ragged M and N edges) split K
])
def test_gemm_mx_small(dev, stream, prec, m, n, k, awq):
    q, xb = problem(m, n, k, 7 * m + n, awq)
    got = run(dev, stream, q, xb, prec)
    check_exact(got, operand(xb, q, prec), q, f"m={m} n={n} k={k} awq={awq}")


@pytest.mark.parametrize("m,n,k", [(512, 9728, 2560), (512, 2560, 9728), (2048, 9728, 2560), (2048, 2560, 9728)])
def test_gemm_mx_configs3(dev, stream, m, n, k):
    """BASELINE configs[3] at its full sizes: X bf16 N(0,1), W INT4 g128 from N(0,0.02), bf16
    out; the fp8-e4m3 variant against the bf16 result and the CPU path."""
    print(f"gemm bf16/fp8 configs[3] m={m} n={n} k={k}", flush=True)
    q, xb = problem(m, n, k, 3 * m + k, False)
    yb = run(dev, stream, q, xb, ops.GEMM_BF16)
    check_exact(yb, operand(xb, q, ops.GEMM_BF16), q, f"bf16 m={m} n={n}")
    y8 = run(dev, stream, q, xb, ops.GEMM_FP8_E4M3)
    check_exact(y8, operand(xb, q, ops.GEMM_FP8_E4M3), q, f"fp8 m={m} n={n}")
    # the reference's CPU path: f16 dequantized weights, f32 matvec (x exact in f16 here)
    wdq = O.dequant_affine_int4(q.data, q.scales_f32, q.zeros_f32, n, k)
    x16 = O.bf16_to_f32(xb).astype(np.float16)
    ref = O.matvec_f16w(wdq, x16, None, nthreads=16)
    rb, r8, r8b = rel_l2(yb, ref), rel_l2(y8, ref), rel_l2(y8, yb)
    print(f"  rel-L2 vs CPU path: bf16 {rb:.2e}  fp8 {r8:.2e};  fp8 vs bf16 {r8b:.2e}", flush=True)
    assert rb <= 3e-3
    assert r8 <= 5e-2 and r8b <= 5e-2


def test_gemm_mx_f16_is_the_projection(dev, stream):
    """IMH_GEMM_F16 runs the projection op (f16 in and out)."""
    rng = np.random.default_rng(5)
    q = quant.quantize_int4((rng.standard_normal((512, 1024)) * 0.02).astype(np.float32))
    x16 = rng.standard_normal((40, 1024)).astype(np.float16)
    wt = ops.AffineQuantizedWeight(dev, q)
    xd = dev.upload(x16)
    a, b = dev.empty((40, 512), np.float16), dev.empty((40, 512), np.float16)
    ops.encode_affine_gemm_int4(stream, xd, 40, wt, a, ops.GEMM_F16)
    ops.encode_projection(stream, xd, wt, b, 40)
    stream.sync()
    assert np.array_equal(a.read().view(np.uint16), b.read().view(np.uint16))


def test_gemm_mx_errors(dev, stream):
    from ironmill_amd import IronmillError
    rng = np.random.default_rng(6)
    wt = ops.AffineQuantizedWeight(dev, quant.quantize_int4((rng.standard_normal((64, 256)) * 0.02).astype(np.float32)))
    x = dev.empty((4, 256), np.uint16)
    y = dev.empty((4, 64), np.uint16)
    with pytest.raises(IronmillError, match="unknown precision"):
        ops.encode_affine_gemm_int4(stream, x, 4, wt, y, 7)
