"""GPU parity of the INT8 weight matvec and the INT4 x Q8 decode variant.

INT8 weights (imh_encode_affine_projection_int8; superblock_matvec_int8,
affine_matvec.metal:123-189, over quantize_tensor_int8, quantized.rs:852-901):

* against the kernel's arithmetic restated exactly: a = x / awq (f32) times the
  exact weights (q - z16) * s16, summed in float64.  The GPU carries a as f16
  hi + lo (~22 bits) and sums in f32, then rounds to f16, so it must be within
  one f16 step of that value plus 2^-18 of sum_k |a| (q + |z|) s (the per-group
  form s * (sum a q - z sum a) cancels terms of that size);
* against the reference's CPU path (dequantize to f16 with f32 params, f32
  matvec): the north star's rel-L2 <= 1e-3.

Q8 activations (imh_encode_quantize_input_q8, quantize.metal:21-52): the codes
and scales are integer / IEEE-exact work and must equal the oracle bit for bit.

INT4 x Q8 (imh_encode_affine_matvec_int4xq8, affine_fused.metal:115-176): the
group sums are exact integers on the GPU (int32 MFMA), so the result must be
the oracle's exact value (integer group sums, f64) up to the f32 scale products
(2^-20 of sum_g |ws as d_g|) and one f16 step.  Against the plain f16 path
(no Q8) the error is the Q8 rounding itself: per element up to absmax / 254,
~0.7 % RMS of a Gaussian row, so rel-L2 <= 2e-2 there.
"""
import numpy as np
import pytest

import oracle as O
from conftest import rel_l2
from ironmill_amd import IronmillError, ops, quant

pytestmark = pytest.mark.gpu


def f16_step(v):
    mag = np.maximum(np.abs(v), 2.0 ** -14)
    return np.exp2(np.floor(np.log2(mag)) - 10)


def int8_problem(n, k, b, seed, awq):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    s = rng.uniform(0.5, 2.0, k).astype(np.float32) if awq else None
    x = rng.standard_normal((b, k)).astype(np.float16)
    return quant.quantize_int8(w, awq_scales=s), x


@pytest.mark.parametrize("n,k,b,awq", [
    (64, 128, 1, False),       # one group, one workgroup
    (1000, 1024, 3, True),     # ragged N, AWQ
    (1000, 1024, 11, True),    # two launches of batch rows (8 + 3)
    (2560, 9728, 1, False),    # Qwen3-4B down shape (sensitive layer in INT8): band kernel, 2-tile bands
    (2560, 9728, 2, True),     # band kernel, two batch rows
    (2560, 9728, 3, False),    # band kernel, 127 KB of LDS
    (2560, 9728, 4, False),    # image too large for the band kernel: tile kernel
    (9728, 2560, 4, True),     # band kernel, 5-tile bands, four batch rows
    (300, 5120, 1, False),     # band kernel, fewer bands than compute units
    (9728, 2560, 8, False),    # gate / up shape, batch 8
    (9728, 256, 2, False),     # band kernel with fewer threads (64) than outputs (80): looped epilogue
    (9728, 256, 4, True),      # one wave against 160 outputs per band
])
def test_int8_projection(dev, stream, n, k, b, awq):
    print(f"int8 projection n={n} k={k} b={b} awq={awq}", flush=True)
    q, x = int8_problem(n, k, b, 11 * n + k + b, awq)
    wt = ops.AffineInt8Weight(dev, q)
    y = dev.empty((b, n), np.float16)
    ops.encode_projection_int8(stream, dev.upload(x), wt, y, b)
    stream.sync()
    got = y.read().astype(np.float64)

    a = x.astype(np.float32)
    if q.awq is not None:
        a = (a / q.awq.astype(np.float32)).astype(np.float32)
    a = a.astype(np.float64)
    s = q.scales.astype(np.float64).repeat(128, axis=1)
    z = q.zeros.astype(np.float64).repeat(128, axis=1)
    codes = q.data.astype(np.float64)
    exact = a @ ((codes - z) * s).T
    terms = np.abs(a) @ ((codes + np.abs(z)) * s).T
    worst = float(np.max(np.abs(got - exact) / (f16_step(exact) + 2.0 ** -18 * terms)))
    assert worst <= 1.0, f"worst error {worst:.2f} x (f16 step + 2^-18 terms)"

    wdq = O.dequant_affine_int8(q.data, q.scales_f32, q.zeros_f32, n, k)
    ref = O.matvec_f16w(wdq, x, q.awq, nthreads=16)
    assert rel_l2(got, ref) <= 1e-3


@pytest.mark.parametrize("t,k", [(1, 128), (1, 2560), (5, 9728), (64, 4096)])
def test_quantize_input_q8_bit_exact(dev, stream, t, k):
    rng = np.random.default_rng(t * 7 + k)
    x = (rng.standard_normal((t, k)) * 3.0).astype(np.float16)
    x[0, :128] = 0.0                                        # all-zero group
    if k > 128:
        x[0, 128:256] = rng.integers(-127, 128, 128).astype(np.float16)
    q8d, scd = dev.empty((t, k), np.int8), dev.empty((t, k // 128), np.float32)
    ops.encode_quantize_input_q8(stream, dev.upload(x), t, k, q8d, scd)
    stream.sync()
    q8, sc = O.quantize_input_q8(x)
    assert np.array_equal(q8d.read(), q8)
    assert np.array_equal(scd.read().view(np.uint32), sc.view(np.uint32))


@pytest.mark.parametrize("n,k,t", [
    (64, 128, 1),              # band kernel, one group (odd: the pair's second half is empty)
    (300, 1152, 3),            # band kernel, 9 groups, fewer bands than compute units
    (1000, 1024, 5),           # ragged N
    (9728, 2560, 8),           # band kernel, 5-tile bands, eight batch rows
    (4096, 2560, 16),          # q_proj, one full token tile
    (1000, 1024, 17),          # two token tiles, ragged
    (9728, 2560, 1),           # gate / up
    (2560, 9728, 1),           # down
    (3072, 1024, 8),           # Qwen3-0.6B gate / up: one wave against 128 outputs per band
    (30000, 1024, 8),          # tall matrix, 5-tile bands: two waves against 320 outputs per band
])
def test_int4xq8_matvec(dev, stream, n, k, t):
    print(f"int4xq8 n={n} k={k} t={t}", flush=True)
    rng = np.random.default_rng(n + k + 3 * t)
    q = quant.quantize_int4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((t, k)).astype(np.float16)
    wt = ops.AffineQuantizedWeight(dev, q)
    q8d, scd = dev.empty((t, k), np.int8), dev.empty((t, k // 128), np.float32)
    y = dev.empty((t, n), np.float16)
    ops.encode_quantize_input_q8(stream, dev.upload(x), t, k, q8d, scd)
    ops.encode_affine_matvec_int4xq8(stream, q8d, scd, t, wt, y)
    stream.sync()
    got = y.read().astype(np.float64)

    q8, sc = O.quantize_input_q8(x)
    exact = O.matvec_int4xq8(q8, sc, q.data, q.scales, q.zeros, n, k)
    codes = O.unpack_int4(q.data.reshape(-1), n * k).reshape(n, k // 128, 128).astype(np.float64)
    zr = np.rint(q.zeros.astype(np.float64))[:, :, None]
    # |ws * as * d_g| summed over groups, d_g the exact integer group sum
    d = np.einsum("tgi,ngi->tng", q8.reshape(t, k // 128, 128).astype(np.float64), codes - zr)
    terms = np.abs(d * sc[:, None, :] * q.scales.astype(np.float64)[None, :, :]).sum(axis=2)
    worst = float(np.max(np.abs(got - exact) / (f16_step(exact) + 2.0 ** -20 * terms)))
    assert worst <= 1.0, f"worst error {worst:.2f} x (f16 step + 2^-20 terms)"

    wdq = O.dequant_affine_int4(q.data, q.scales_f32, q.zeros_f32, n, k)
    ref = O.matvec_f16w(wdq, x, None, nthreads=16)
    r = rel_l2(got, ref)
    print(f"  rel-L2 vs the f16 path (Q8 rounding): {r:.2e}", flush=True)
    assert r <= 2e-2


@pytest.mark.parametrize("n,k,t,codes", [
    (9728, 2560, 1, True),     # gate / up shape, codes written for reuse
    (9728, 2560, 1, False),
    (2560, 9728, 1, True),     # down shape
    (4096, 2560, 8, True),     # eight rows
    (3072, 1024, 8, False),    # fewer threads than outputs per band
    (64, 128, 3, True),        # one group
    (1000, 1024, 11, True),    # above 8 rows: the two launches, codes in the caller's buffers
    (1000, 1024, 11, False),   # the two launches, codes in scratch memory
])
def test_projection_int4_q8_one_launch(dev, stream, n, k, t, codes):
    """imh_encode_affine_projection_int4_q8 quantizes the f16 rows while it stages them: y
    equals the quantize + matvec launches bit for bit, and the codes / scales it writes equal
    imh_encode_quantize_input_q8's (bit-exact with the oracle)."""
    print(f"int4 q8 one launch n={n} k={k} t={t} codes={codes}", flush=True)
    rng = np.random.default_rng(3 * n + k + t)
    q = quant.quantize_int4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((t, k)).astype(np.float16)
    x[0, :128] = 0.0                                        # an all-zero group
    wt = ops.AffineQuantizedWeight(dev, q)
    xd = dev.upload(x)
    q8d, scd = dev.empty((t, k), np.int8), dev.empty((t, k // 128), np.float32)
    y2 = dev.empty((t, n), np.float16)
    ops.encode_quantize_input_q8(stream, xd, t, k, q8d, scd)
    ops.encode_affine_matvec_int4xq8(stream, q8d, scd, t, wt, y2)
    y1 = dev.empty((t, n), np.float16)
    q8o = dev.empty((t, k), np.int8) if codes else None
    sco = dev.empty((t, k // 128), np.float32) if codes else None
    ops.encode_projection_int4_q8(stream, xd, wt, y1, t, q8o, sco)
    stream.sync()
    assert np.array_equal(y1.read().view(np.uint16), y2.read().view(np.uint16))
    if codes:
        q8, sc = O.quantize_input_q8(x)
        assert np.array_equal(q8o.read(), q8)
        assert np.array_equal(sco.read().view(np.uint32), sc.view(np.uint32))


def test_int8_q8_errors(dev, stream):
    rng = np.random.default_rng(9)
    q = quant.quantize_int4((rng.standard_normal((64, 256)) * 0.02).astype(np.float32),
                            awq_scales=rng.uniform(0.5, 2, 256).astype(np.float32))
    wt = ops.AffineQuantizedWeight(dev, q)
    q8, sc, y = dev.empty((1, 256), np.int8), dev.empty((1, 2), np.float32), dev.empty((1, 64), np.float16)
    with pytest.raises(IronmillError, match="no AWQ"):
        ops.encode_affine_matvec_int4xq8(stream, q8, sc, 1, wt, y)
    with pytest.raises(IronmillError, match="multiple of 128"):
        ops.encode_quantize_input_q8(stream, dev.empty((1, 200), np.float16), 1, 200, q8, sc)
    with pytest.raises(IronmillError, match="no AWQ"):
        ops.encode_projection_int4_q8(stream, dev.empty((1, 256), np.float16), wt, y, 1)
    plain = ops.AffineQuantizedWeight(dev, quant.quantize_int4((rng.standard_normal((64, 256)) * 0.02)
                                                               .astype(np.float32)))
    with pytest.raises(IronmillError, match="both given or both NULL"):
        ops.encode_projection_int4_q8(stream, dev.empty((1, 256), np.float16), plain, y, 1, q8_out=q8)
