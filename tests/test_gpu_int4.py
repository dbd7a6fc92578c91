"""GPU parity of the INT4 affine ops against the CPU oracle, through the C ABI.

The expected values come from the oracle's own chain -- quantize_tensor_int4
(quantized.rs:408-465) -> dequant_affine with f32 params (core/dequant.rs:85-180)
-> f32-accumulate dot -- on the same seeded inputs; the GPU gets its weights
from the library's host quantizer, so a mismatch in either shows up here.
Tolerance: rel-L2 <= 1e-3 and max-abs <= 2e-2 on
the f16 outputs.
"""
import numpy as np
import pytest

import oracle as O
from conftest import assert_close
from ironmill_amd import IronmillError, ops, quant

pytestmark = pytest.mark.gpu


def make_weight(n, k, seed, awq=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16).astype(np.float32)
    s = rng.uniform(0.5, 2.0, k).astype(np.float32) if awq else None
    return w, s


def make_x(batch, k, seed, outliers=True):
    rng = np.random.default_rng(seed + 1000)
    x = rng.standard_normal((batch, k)).astype(np.float32)
    if outliers:  # 1 % of channels x20
        idx = rng.choice(k, max(1, k // 100), replace=False)
        x[:, idx] *= 20.0
    return x.astype(np.float16)


def oracle_dense(w, s):
    """Oracle quantize + CPU dequant -> dense f16 W and the f16 AWQ vector."""
    wq = w if s is None else (w * s[None, :]).astype(np.float32)
    packed, sc, zp = O.quantize_tensor_int4(wq, 128)
    n, k = w.shape
    wdq = O.dequant_affine_int4(packed, sc, zp, n, k, 128)
    awq16 = None if s is None else s.astype(np.float16)
    return wdq, awq16


def upload_weight(dev, w, s):
    return ops.AffineQuantizedWeight(dev, quant.quantize_int4(w, awq_scales=s))


def gpu_layout_y(q, x16, awq16=None):
    """y of the GPU weight layout in float64: fp16 scales/zeros (the reference's
    upload, metal/weights.rs:1064-1092), exact (q - z) * s, f32 x / awq."""
    codes = np.stack([q.data & 0x0F, q.data >> 4], axis=-1).reshape(q.n, q.k).astype(np.float64)
    s = np.repeat(q.scales.astype(np.float64), 128, axis=1)
    z = np.repeat(q.zeros.astype(np.float64), 128, axis=1)
    xe = x16.astype(np.float32)
    if awq16 is not None:
        xe = (xe / awq16.astype(np.float32)).astype(np.float32)
    return xe.astype(np.float64) @ ((codes - z) * s).T


@pytest.mark.parametrize("n,k,batch,awq", [
    (1024, 1024, 1, False),
    (1024, 1024, 4, True),
    (1000, 256, 3, False),    # ragged N (not a multiple of 16)
    (64, 128, 17, True),      # one group, batch beyond one 16-row MFMA tile
    (2560, 9728, 1, True),    # Qwen3-4B down projection
    (2560, 9728, 8, True),
    (4096, 2560, 1, False),   # Qwen3-4B Q projection
    (1003, 1024, 2, True),    # batch 2, ragged N (not a multiple of 8)
    (1003, 384, 1, False),    # an odd number of groups
    (24, 256, 1, True),       # one group pair
    (2560, 4096, 1, True),    # Qwen3-4B O projection
    (1024, 2560, 2, False),   # Qwen3-4B K / V projection, batch 2
    (5000, 1024, 1, True),    # bands of 17-24 rows
    (151936 // 8, 2560, 1, False),   # an LM-head-like tall matrix (bands of 3 tiles at 1-2 rows)
    (151936, 2560, 1, False),        # the Qwen3-4B LM head itself at one row
    (15005, 2560, 2, True),          # tall, two rows, a ragged last band
    (151936 // 8, 2560, 4, True),    # 3-8 rows on a tall matrix: one band per CU in 5-tile blocks
    (151936 // 8, 2560, 8, False),
    (15003, 2560, 5, True),          # the same with a ragged last block
    (12000, 1024, 8, True),          # one group pair per wave
    (151936, 2560, 8, False),        # the Qwen3-4B LM head at 8 rows
    # 3-8 rows with fewer 16-row tiles than compute units: split-K over K slices
    (2560, 9728, 3, False),
    (2560, 4096, 4, False),          # 32 groups, the fewest split
    (1000, 9728, 6, True),           # ragged N, 13 bands
    (2000, 5248, 5, True),           # 41 groups: slices of 5-6
    (1024, 32768, 7, True),          # 256 groups: 16 waves of 2 groups per slice
])
def test_projection_matches_oracle(dev, stream, n, k, batch, awq):
    w, s = make_weight(n, k, seed=n + k + batch, awq=awq)
    x16 = make_x(batch, k, seed=n * 7 + k)
    wt = upload_weight(dev, w, s)
    xd = dev.upload(x16)
    yd = dev.empty((batch, n), np.float16)
    ops.encode_projection(stream, xd, wt, yd, batch)
    stream.sync()
    got = yd.read()
    wdq, awq16 = oracle_dense(w, s)
    ref = O.matvec_f16w(wdq, x16, awq16, nthreads=8)
    assert_close(got, ref, what=f"projection n={n} k={k} B={batch} awq={awq}", ulps=2)
    lay = gpu_layout_y(quant.quantize_int4(w, awq_scales=s), x16, awq16)
    assert_close(got, lay, what="projection vs GPU-layout semantics")


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_fused_gate_up_qwen_shape(dev, stream, batch, act):
    n, k = 9728, 2560
    wg, s = make_weight(n, k, seed=11, awq=True)
    wu, _ = make_weight(n, k, seed=12, awq=False)
    x16 = make_x(batch, k, seed=13 + batch)
    q_up = quant.quantize_int4(wu, awq_scales=s)  # gate's AWQ divides x for both (ops/quantized.rs:218-224)
    gate = upload_weight(dev, wg, s)
    up = ops.AffineQuantizedWeight(dev, q_up)
    xd = dev.upload(x16)
    out = dev.empty((batch, n), np.float16)
    ops.encode_fused_ffn_gate_up_act_int4(stream, xd, gate, up, out, batch, use_gelu=(act == "gelu"))
    stream.sync()
    wdq_g, awq16 = oracle_dense(wg, s)
    wdq_u, _ = oracle_dense(wu, s)
    ref = O.gate_up_act(wdq_g, wdq_u, x16, awq16, act=act)
    assert_close(out.read(), ref, what=f"fused gate+up {act} B={batch}", ulps=2)


def _ffn_case(dev, n, k, batch, seed, down_awq=True):
    wg, s = make_weight(n, k, seed=seed, awq=True)
    wu, _ = make_weight(n, k, seed=seed + 1)
    wd, sd = make_weight(k, n, seed=seed + 2, awq=down_awq)
    x16 = make_x(batch, k, seed=seed + 3 + batch)
    gate = upload_weight(dev, wg, s)
    up = ops.AffineQuantizedWeight(dev, quant.quantize_int4(wu, awq_scales=s))
    down = upload_weight(dev, wd, sd)
    return (wg, wu, wd, s, sd, x16), (gate, up, down)


@pytest.mark.parametrize("n,k,batch,act,down_awq", [
    (9728, 2560, 1, "silu", True),    # Qwen3-4B FFN
    (9728, 2560, 1, "gelu", True),
    (9728, 2560, 2, "silu", False),   # down without AWQ scales
    (512, 256, 2, "silu", True),
    (1280, 256, 1, "silu", True),     # 5-row bands (odd starts): no operand image, two plain ops
    (9728, 2560, 4, "silu", True),    # 3-8 rows: the image into the tile kernel (no prep launch)
    (9728, 2560, 8, "gelu", False),
    (10240, 2560, 1, "silu", True),   # Qwen3.5-4B intermediate size
    (512, 256, 40, "silu", True),     # prefill-sized: the GEMM ops
])
def test_ffn_block_matches_oracle(dev, stream, n, k, batch, act, down_awq):
    """encode_ffn_block: act against the oracle's gate_up_act; y against the
    oracle's down projection of the act the GPU wrote (so act's own rounding is
    not counted twice); the same act as the fused gate+up op, bit for bit, and
    y bit for bit that of the two ops -- at 1-8 rows the gate/up launch hands
    down its operand image (the same per-element arithmetic, done once instead
    of in every down workgroup or a prep launch)."""
    (wg, wu, wd, s, sd, x16), (gate, up, down) = _ffn_case(dev, n, k, batch, seed=21, down_awq=down_awq)
    xd = dev.upload(x16)
    act_d = dev.empty((batch, n), np.float16)
    y = dev.empty((batch, k), np.float16)
    gelu = act == "gelu"
    ops.encode_ffn_block_int4(stream, xd, gate, up, down, act_d, y, batch, use_gelu=gelu)
    stream.sync()
    got_act, got_y = act_d.read(), y.read()
    wdq_g, awq16 = oracle_dense(wg, s)
    wdq_u, _ = oracle_dense(wu, s)
    assert_close(got_act, O.gate_up_act(wdq_g, wdq_u, x16, awq16, act=act), what="ffn act", ulps=2)
    wdq_d, awqd = oracle_dense(wd, sd)
    assert_close(got_y, O.matvec_f16w(wdq_d, got_act, awqd, nthreads=8), what="ffn y", ulps=2)
    # the two ops on the same inputs
    act2 = dev.empty((batch, n), np.float16)
    y2 = dev.empty((batch, k), np.float16)
    ops.encode_fused_ffn_gate_up_act_int4(stream, xd, gate, up, act2, batch, use_gelu=gelu)
    ops.encode_projection(stream, act2, down, y2, batch)
    stream.sync()
    assert np.array_equal(act2.read().view(np.uint16), got_act.view(np.uint16)), "act differs from the fused op"
    # the block's down reads the operand image gate/up wrote (1-8 rows) with the two
    # ops' per-element arithmetic, or runs the two ops: bit for bit either way
    assert np.array_equal(y2.read().view(np.uint16), got_y.view(np.uint16)), "y differs from the two ops"


def test_ffn_block_repeated_launches(dev, stream):
    """Back-to-back FFN blocks of different shapes on one stream, then a graph
    replaying one (with eager work between the replays), give the eager result
    every time."""
    big = _ffn_case(dev, 9728, 2560, 1, seed=31)
    small = _ffn_case(dev, 512, 256, 2, seed=41)
    outs = {}
    for name, ((*_, x16), (gate, up, down)), b in (("big", big, 1), ("small", small, 2)):
        xd = dev.upload(x16)
        a = dev.empty((b, gate.n), np.float16)
        y = dev.empty((b, gate.k), np.float16)
        outs[name] = (xd, gate, up, down, a, y, b)
    ref = {}
    for it in range(3):
        for name in ("big", "small", "big"):
            xd, gate, up, down, a, y, b = outs[name]
            ops.encode_ffn_block_int4(stream, xd, gate, up, down, a, y, b)
            stream.sync()
            got = y.read().view(np.uint16).copy()
            if name not in ref:
                ref[name] = got
            assert np.array_equal(got, ref[name]), f"launch {it} {name}"
    xd, gate, up, down, a, y, b = outs["big"]
    graph = stream.capture(lambda: [ops.encode_ffn_block_int4(stream, xd, gate, up, down, a, y, b)
                                    for _ in range(4)])
    for rep in range(3):
        y.write(np.zeros((b, gate.k), np.float16))
        graph.launch(stream)
        stream.sync()
        assert np.array_equal(y.read().view(np.uint16), ref["big"]), f"graph replay {rep}"
        ops.encode_ffn_block_int4(stream, *outs["small"][:6], 2)   # eager work between replays
        stream.sync()


@pytest.mark.parametrize("batch,awq", [(1, True), (2, False), (8, False)])
def test_batched_gate_up(dev, stream, batch, awq):
    n, k = 9728, 2560
    wg, s = make_weight(n, k, seed=21, awq=awq)
    wu, _ = make_weight(n, k, seed=22)
    x16 = make_x(batch, k, seed=23)
    gate = upload_weight(dev, wg, s)
    up = ops.AffineQuantizedWeight(dev, quant.quantize_int4(wu, awq_scales=s))
    xd = dev.upload(x16)
    go, uo = dev.empty((batch, n), np.float16), dev.empty((batch, n), np.float16)
    ops.encode_batched_affine_matvec_int4(stream, xd, gate, go, up, uo, batch)
    stream.sync()
    wdq_g, awq16 = oracle_dense(wg, s)
    wdq_u, _ = oracle_dense(wu, s)
    assert_close(go.read(), O.matvec_f16w(wdq_g, x16, awq16, nthreads=8), what="gate", ulps=2)
    assert_close(uo.read(), O.matvec_f16w(wdq_u, x16, awq16, nthreads=8), what="up", ulps=2)


# 3-8 rows: the residual + norm prep kernel at 1, 2 and 8 register chunks per
# thread, and past those (K > 16384: the chunks beyond are read again)
@pytest.mark.parametrize("n,k,batch,awq", [
    (4096, 2560, 1, False), (4096, 2560, 1, True), (4096, 2560, 2, True), (4096, 2560, 3, True),
    (4096, 2560, 8, False), (512, 1024, 5, True), (128, 16384, 4, False), (128, 16512, 3, True),
])
def test_fused_residual_norm_projection(dev, stream, n, k, batch, awq):
    eps = 1e-6
    w, s = make_weight(n, k, seed=31, awq=awq)
    rng = np.random.default_rng(32)
    a = rng.standard_normal((batch, k)).astype(np.float16)
    b = (rng.standard_normal((batch, k)) * 0.5).astype(np.float16)
    gamma = rng.uniform(0.5, 1.5, k).astype(np.float16)
    wt = upload_weight(dev, w, s)
    ad, bd, gd = dev.upload(a), dev.upload(b), dev.upload(gamma)
    y = dev.empty((batch, n), np.float16)
    res = dev.empty((batch, k), np.float16)
    nrm = dev.empty((batch, k), np.float16)
    ops.encode_fused_residual_norm_affine_matvec_int4(stream, ad, bd, gd, res, wt, y, nrm, eps, batch)
    stream.sync()
    wdq, awq16 = oracle_dense(w, s)
    y_ref, res_ref, nrm_ref = O.fused_residual_norm_matvec(a, b, gamma, wdq, eps, awq16)
    assert_close(y.read(), y_ref, what="resnorm y", ulps=2)
    # f16(a + b) is one f32 add and one RNE rounding on both sides: bit-exact
    assert np.array_equal(res.read().view(np.uint16), res_ref.view(np.uint16))
    assert_close(nrm.read(), nrm_ref.astype(np.float32), rel=1e-3, max_abs=2e-3, what="normed")


# The kernels apply the zero point per group as s * (sum x q - z * sum x), with
# both sums in f32, so the closed forms below hold to f32 rounding of those
# sums (|error| ~ 2^-24 * 8 * sum |x| * s per group), not to the last bit.
CLOSED_FORM_ATOL = 1e-4


def test_codes_equal_to_zero_point_give_zero(dev, stream):
    """Closed form: q == z everywhere -> (q - z) * s == 0, so y == 0."""
    n, k = 256, 1024
    q = quant.QuantizedInt4(
        data=np.full((n, k // 2), 0x77, np.uint8),
        scales=np.full((n, k // 128), 0.01, np.float16), zeros=np.full((n, k // 128), 7.0, np.float16),
        scales_f32=None, zeros_f32=None, awq=None, n=n, k=k)
    wt = ops.AffineQuantizedWeight(dev, q)
    x16 = make_x(4, k, seed=5)
    xd, yd = dev.upload(x16), dev.empty((4, n), np.float16)
    ops.encode_projection(stream, xd, wt, yd, 4)
    stream.sync()
    assert np.abs(yd.read().astype(np.float32)).max() <= CLOSED_FORM_ATOL


def test_single_nibble_picks_one_column(dev, stream):
    """Closed form: one code differs from z by d at (r, c) -> y[r] = x[c] * d * s."""
    n, k = 32, 256
    codes = np.full((n, k), 8, np.uint8)
    codes[5, 77] = 11   # +3 steps
    codes[20, 200] = 2  # -6 steps
    data = (codes[:, 1::2] << 4 | codes[:, 0::2]).astype(np.uint8)
    q = quant.QuantizedInt4(data=data, scales=np.full((n, 2), 0.25, np.float16),
                            zeros=np.full((n, 2), 8.0, np.float16), scales_f32=None, zeros_f32=None,
                            awq=None, n=n, k=k)
    wt = ops.AffineQuantizedWeight(dev, q)
    x16 = make_x(1, k, seed=9, outliers=False)
    xd, yd = dev.upload(x16), dev.empty((1, n), np.float16)
    ops.encode_projection(stream, xd, wt, yd, 1)
    stream.sync()
    exp = np.zeros(n, np.float32)
    exp[5] = np.float32(x16[0, 77]) * 3 * 0.25
    exp[20] = np.float32(x16[0, 200]) * -6 * 0.25
    got = yd.read()[0].astype(np.float32)
    exp16 = exp.astype(np.float16).astype(np.float32)
    ulp = np.spacing(np.abs(exp16).astype(np.float16)).astype(np.float32)
    assert np.all(np.abs(got - exp16) <= np.maximum(CLOSED_FORM_ATOL, ulp))


def test_error_paths(dev, stream):
    w, _ = make_weight(64, 256, seed=1)
    wt = upload_weight(dev, w, None)
    bad = ops.AffineQuantizedWeight.from_pointers(wt.data, wt.scales, wt.zeros, None, 64, 256, 64)
    xd, yd = dev.upload(make_x(1, 256, 2)), dev.empty((1, 64), np.float16)
    with pytest.raises(IronmillError, match="group_size"):
        ops.encode_projection(stream, xd, bad, yd, 1)
    bad_k = ops.AffineQuantizedWeight.from_pointers(wt.data, wt.scales, wt.zeros, None, 64, 200, 128)
    with pytest.raises(IronmillError, match="multiple of 128"):
        ops.encode_projection(stream, xd, bad_k, yd, 1)
    other = ops.AffineQuantizedWeight.from_pointers(wt.data, wt.scales, wt.zeros, None, 32, 256, 128)
    with pytest.raises(IronmillError, match="shapes differ"):
        ops.encode_fused_ffn_gate_up_act_int4(stream, xd, wt, other, yd, 1)
    ops.encode_projection(stream, xd, wt, yd, 0)  # zero tokens: no-op
    stream.sync()
