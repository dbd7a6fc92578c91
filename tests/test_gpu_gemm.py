"""GPU parity of the INT4 ops at prefill-sized token counts (the GEMM path:
superblock_matmul_int4, affine_matmul.metal:10-152, reached through
encode_projection at token_count > 1, projection.rs:227-312) against the CPU
oracle's dequantize-then-compute chain.

The GEMM multiplies the exact weight (the code minus its zero point in f16,
the f16 scale applied per group in f32) with x (exact f16) or, with AWQ,
with x / awq carried as f16 hi + lo (~22 bits; rounding it to f16 alone,
as the reference's prefill kernel does, moves outputs by several fp16 steps
where terms cancel).  Tolerance as on the decode path: rel-L2 <= 1e-3
and max-abs <= max(2e-2, 2 fp16 steps of the reference value)
(f16 scales on the GPU, f32 on the CPU path: one step, plus the output
rounding).
"""
import numpy as np
import pytest

import oracle as O
from conftest import assert_close
from ironmill_amd import ops, quant

pytestmark = pytest.mark.gpu


def ulps_for(awq):
    return 2


def weight(n, k, seed, awq):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16).astype(np.float32)
    s = rng.uniform(0.5, 2.0, k).astype(np.float32) if awq else None
    return w, s


def acts(m, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    idx = rng.choice(k, max(1, k // 100), replace=False)
    x[:, idx] *= 20.0
    return x.astype(np.float16)


def exact_weights(q):
    """The uploaded weight exactly, in f64: f16 scale x (code - f16 zero point)."""
    codes = np.empty((q.n, q.k), np.float64)
    codes[:, 0::2] = q.data & 0xF
    codes[:, 1::2] = q.data >> 4
    sc = np.repeat(q.scales.astype(np.float64), q.group_size, axis=1)
    zp = np.repeat(q.zeros.astype(np.float64), q.group_size, axis=1)
    return sc * (codes - zp)


def dense(w, s):
    wq = w if s is None else (w * s[None, :]).astype(np.float32)
    packed, sc, zp = O.quantize_tensor_int4(wq, 128)
    n, k = w.shape
    return O.dequant_affine_int4(packed, sc, zp, n, k, 128), (None if s is None else s.astype(np.float16))


@pytest.mark.parametrize("m,n,k,awq", [
    (32, 1000, 256, False),    # smallest GEMM token count, ragged N
    (64, 2560, 9728, True),    # Qwen3-4B down, split-K
    (200, 1000, 256, False),   # ragged M and N, one K split
    (128, 9728, 2560, True),   # Qwen3-4B gate shape, split-K over 76 x 1 tiles
    (512, 1024, 2560, True),   # BASELINE configs[3] M, smaller N
])
def test_gemm_projection(dev, stream, m, n, k, awq):
    w, s = weight(n, k, m + n, awq)
    x16 = acts(m, k, 3 * m + k)
    wt = ops.AffineQuantizedWeight(dev, quant.quantize_int4(w, awq_scales=s))
    xd, yd = dev.upload(x16), dev.empty((m, n), np.float16)
    ops.encode_projection(stream, xd, wt, yd, m)
    stream.sync()
    wdq, awq16 = dense(w, s)
    ref = O.matvec_f16w(wdq, x16, awq16, nthreads=8)
    assert_close(yd.read(), ref, what=f"gemm m={m} n={n} k={k} awq={awq}", ulps=ulps_for(awq))


@pytest.mark.parametrize("m,n,k", [(512, 9728, 2560), (512, 2560, 9728), (2048, 9728, 2560), (2048, 2560, 9728)])
def test_gemm_configs3_full_shapes(dev, stream, m, n, k):
    """BASELINE configs[3] at its full sizes (M = 512 / 2048, (K, N) = (2560, 9728) and
    (9728, 2560)), AWQ, every output against the oracle."""
    print(f"gemm configs[3] m={m} n={n} k={k}", flush=True)
    w, s = weight(n, k, 7 * m + n, True)
    x16 = acts(m, k, 11 * m + k)
    wt = ops.AffineQuantizedWeight(dev, quant.quantize_int4(w, awq_scales=s))
    xd, yd = dev.upload(x16), dev.empty((m, n), np.float16)
    ops.encode_projection(stream, xd, wt, yd, m)
    stream.sync()
    wdq, awq16 = dense(w, s)
    ref = O.matvec_f16w(wdq, x16, awq16, nthreads=16)
    assert_close(yd.read(), ref, what=f"gemm m={m} n={n} k={k}", ulps=ulps_for(True))


def test_gemm_matches_matvec_at_the_switch(dev, stream):
    """The same rows through the matvec (31 tokens) and the GEMM (32 tokens)."""
    n, k = 512, 1024
    w, s = weight(n, k, 5, True)
    wt = ops.AffineQuantizedWeight(dev, quant.quantize_int4(w, awq_scales=s))
    x16 = acts(32, k, 6)
    y31, y32 = dev.empty((31, n), np.float16), dev.empty((32, n), np.float16)
    ops.encode_projection(stream, dev.upload(x16[:31].copy()), wt, y31, 31)
    ops.encode_projection(stream, dev.upload(x16), wt, y32, 32)
    stream.sync()
    assert_close(y32.read()[:31], y31.read().astype(np.float32), what="gemm vs matvec", ulps=ulps_for(True))


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_gemm_fused_gate_up(dev, stream, act):
    m, n, k = 48, 9728, 2560
    wg, s = weight(n, k, 41, True)
    wu, _ = weight(n, k, 42, False)
    x16 = acts(m, k, 43)
    gate = ops.AffineQuantizedWeight(dev, quant.quantize_int4(wg, awq_scales=s))
    up = ops.AffineQuantizedWeight(dev, quant.quantize_int4(wu, awq_scales=s))
    xd, out = dev.upload(x16), dev.empty((m, n), np.float16)
    ops.encode_fused_ffn_gate_up_act_int4(stream, xd, gate, up, out, m, use_gelu=(act == "gelu"))
    stream.sync()
    got = out.read().astype(np.float64)
    wdq_g, awq16 = dense(wg, s)
    wdq_u, _ = dense(wu, s)
    ref = O.gate_up_act(wdq_g, wdq_u, x16, awq16, act=act)
    assert_close(got, ref, what=f"gemm fused gate+up {act} vs the CPU path", max_abs=np.inf)
    # Element-wise against the exact value of what the kernel computes: the
    # uploaded codes with their f16 scales and zero points, x / awq unrounded,
    # in f64.  The CPU path rounds each dequantized weight to f16; act(gate) *
    # up amplifies that, and at this shape it alone moves an output ~5 f16
    # steps (row 31, column 8523: exact -6.9241, CPU path -6.9079, 0.98 of
    # max(2e-2, 2 steps)), so the bound there would pass or fail on the
    # rounding direction of a correct result.  Bound: 2 f16 steps of the exact
    # value, plus 2^-16 of the summed magnitudes the f32 accumulation and the
    # hi / lo split of x / awq see, carried through act(gate) * up.
    qg = quant.quantize_int4(wg, awq_scales=s)
    qu = quant.quantize_int4(wu, awq_scales=s)
    xa = x16.astype(np.float64) / s.astype(np.float16).astype(np.float64)[None, :]
    Wg, Wu = exact_weights(qg), exact_weights(qu)
    g, u = xa @ Wg.T, xa @ Wu.T
    mg, mu = np.abs(xa) @ np.abs(Wg).T, np.abs(xa) @ np.abs(Wu).T
    if act == "silu":
        a = g / (1.0 + np.exp(-g))
    else:
        a = 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3)))
    exact = a * u
    slack = 2.0 ** -16 * 1.1 * (np.abs(u) * mg + np.abs(a) * mu)
    bound = 2.0 * np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64) + slack
    err = np.abs(got - exact)
    worst = np.unravel_index(np.argmax(err / bound), err.shape)
    assert np.all(err <= bound), (f"gemm fused gate+up {act}: |got - exact| {err[worst]:.3e} > "
                                  f"{bound[worst]:.3e} at {worst} (exact {exact[worst]:.5f}, got {got[worst]:.5f})")


def test_gemm_batched_gate_up(dev, stream):
    m, n, k = 33, 2048, 1024
    wg, s = weight(n, k, 51, True)
    wu, _ = weight(n, k, 52, False)
    x16 = acts(m, k, 53)
    gate = ops.AffineQuantizedWeight(dev, quant.quantize_int4(wg, awq_scales=s))
    up = ops.AffineQuantizedWeight(dev, quant.quantize_int4(wu, awq_scales=s))
    xd = dev.upload(x16)
    go, uo = dev.empty((m, n), np.float16), dev.empty((m, n), np.float16)
    ops.encode_batched_affine_matvec_int4(stream, xd, gate, go, up, uo, m)
    stream.sync()
    wdq_g, awq16 = dense(wg, s)
    wdq_u, _ = dense(wu, s)
    assert_close(go.read(), O.matvec_f16w(wdq_g, x16, awq16, nthreads=8), what="gemm gate", ulps=ulps_for(True))
    assert_close(uo.read(), O.matvec_f16w(wdq_u, x16, awq16, nthreads=8), what="gemm up", ulps=ulps_for(True))


# the residual + norm rows kernel at 1, 2 and 8 register chunks per thread,
# and past those (K > 16384: the chunks beyond are read again)
@pytest.mark.parametrize("m,n,k", [(40, 4096, 2560), (33, 256, 1024), (32, 128, 16384), (34, 128, 16512)])
def test_gemm_fused_residual_norm(dev, stream, m, n, k):
    eps = 1e-6
    w, s = weight(n, k, 61, True)
    rng = np.random.default_rng(62)
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = (rng.standard_normal((m, k)) * 0.5).astype(np.float16)
    gamma = rng.uniform(0.5, 1.5, k).astype(np.float16)
    wt = ops.AffineQuantizedWeight(dev, quant.quantize_int4(w, awq_scales=s))
    ad, bd, gd = dev.upload(a), dev.upload(b), dev.upload(gamma)
    y = dev.empty((m, n), np.float16)
    res = dev.empty((m, k), np.float16)
    nrm = dev.empty((m, k), np.float16)
    ops.encode_fused_residual_norm_affine_matvec_int4(stream, ad, bd, gd, res, wt, y, nrm, eps, m)
    stream.sync()
    wdq, awq16 = dense(w, s)
    y_ref, res_ref, nrm_ref = O.fused_residual_norm_matvec(a, b, gamma, wdq, eps, awq16)
    assert_close(y.read(), y_ref, what="gemm resnorm y", ulps=ulps_for(True))
    assert np.array_equal(res.read().view(np.uint16), res_ref.view(np.uint16))
    assert_close(nrm.read(), nrm_ref.astype(np.float32), rel=1e-3, max_abs=2e-3, what="gemm normed")
