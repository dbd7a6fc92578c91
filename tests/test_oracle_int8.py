"""Pins of the oracle's INT8 weight and Q8 activation restatements (CPU only).

* quantize_tensor_int8 (quantized.rs:852-901): the reference's own test input
  (test_quantize_int8_basic, quantized.rs:1391-1416: a 64 x 128 ramp) with the
  values the mathematics fixes for a ramp (codes 0..255 monotone, scale =
  range / 255), the round-trip bound |w - (q - z) s| <= s / 2 (plus the f32 rounding of
  v / s + z), and the C walk
  against the numpy quantizer of the package on random rows.
* quantize_input_q8 (quantize.metal:21-52): closed forms (an integer group
  whose absmax is 127 has scale 1 and q8 = x; an all-zero group has scale 0 and
  codes 0) and the rounding bound |x - q8 * scale| <= scale / 2.
* matvec_int4xq8 (affine_fused.metal:115-176): on integer activations with
  absmax 127 (so q8 = x exactly) and power-of-two weight scales, it must equal
  the plain f16-weight matvec of the dequantized weights (q - rint(z)) * s; the
  zero-points are set to halves so that using z instead of rint(z) fails.
"""
import numpy as np

import oracle as O
from ironmill_amd import quant


def test_quantize_int8_reference_ramp():
    rows, cols = 64, 128
    w = (np.arange(rows * cols, dtype=np.float32) * np.float32(0.01) - np.float32(40.0)).reshape(rows, cols)
    codes, s, z = O.quantize_tensor_int8(w)
    assert codes.shape == (rows, cols) and codes.dtype == np.uint8   # one byte per value
    for r in range(rows):
        assert codes[r, 0] == 0 and codes[r, -1] == 255
        assert np.all(np.diff(codes[r].astype(int)) >= 0)
        rng = np.float32(w[r].max() - w[r].min())
        assert s[r, 0] == np.float32(rng / np.float32(255.0))
    # the ramp sits far from 0, so z ~ 8000 and v / s + z is formed in f32 (ulp 2^-11 there):
    # half a step plus those roundings
    deq = (codes.astype(np.float64) - z.repeat(128, axis=1)) * s.repeat(128, axis=1)
    assert np.all(np.abs(deq - w) <= s.repeat(128, axis=1) * (0.5 + 2.0 ** -9))


def test_quantize_int8_c_matches_numpy():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((37, 512)) * 0.05).astype(np.float32)
    w[3, 128:256] = 0.25                     # a degenerate (constant) group
    codes, s, z = O.quantize_tensor_int8(w)
    q = quant.quantize_int8(w)
    assert np.array_equal(codes, q.data)
    assert np.array_equal(s, q.scales_f32) and np.array_equal(z, q.zeros_f32)
    d = O.dequant_affine_int8(codes, s, z, 37, 512)
    assert np.max(np.abs(d.astype(np.float64) - w)) <= np.max(s) * 0.5 + 2e-3 * 0.05


def test_quantize_input_q8_closed_forms():
    rng = np.random.default_rng(4)
    k = 512
    x = (rng.standard_normal((3, k)) * 2.0).astype(np.float16)
    x[0, :128] = rng.integers(-127, 128, 128).astype(np.float16)
    x[0, 5] = 127.0                          # absmax exactly 127 -> scale 1
    x[1, 128:256] = 0.0                      # all-zero group
    q8, sc = O.quantize_input_q8(x)
    assert sc[0, 0] == 1.0 and np.array_equal(q8[0, :128].astype(np.float16), x[0, :128])
    assert sc[1, 1] == 0.0 and not np.any(q8[1, 128:256])
    xs = x.astype(np.float64).reshape(3, 4, 128)
    assert np.allclose(sc, np.abs(xs).max(axis=2) / 127.0, rtol=1e-7, atol=0)
    err = np.abs(xs - q8.astype(np.float64).reshape(3, 4, 128) * sc[:, :, None])
    assert np.all(err <= sc[:, :, None] * (0.5 + 1e-5))
    assert q8.min() >= -127


def test_matvec_int4xq8_equals_dense_path_on_exact_inputs():
    rng = np.random.default_rng(5)
    n, k, b = 48, 512, 3
    codes = rng.integers(0, 16, (n, k)).astype(np.uint8)
    packed = O.pack_int4(codes.reshape(-1))
    s16 = np.exp2(rng.integers(-9, -5, (n, k // 128))).astype(np.float16)
    z16 = (rng.integers(2, 13, (n, k // 128)) + 0.5).astype(np.float16)   # halves: rint != z
    x = rng.integers(-127, 128, (b, k)).astype(np.float16)
    x[:, ::128] = 127.0                      # every group's absmax is 127 -> q8 = x, scale 1
    q8, sc = O.quantize_input_q8(x)
    assert np.all(sc == 1.0)
    got = O.matvec_int4xq8(q8, sc, packed, s16, z16, n, k)
    zr = np.rint(z16.astype(np.float32))
    wdq = ((codes.astype(np.float32) - zr.repeat(128, axis=1)) * s16.astype(np.float32).repeat(128, axis=1))
    assert np.array_equal(wdq.astype(np.float16).astype(np.float32), wdq)   # exact in f16
    ref = O.matvec_f16w(wdq.astype(np.float16), x)
    assert np.max(np.abs(got - ref)) <= 1e-6 * np.max(np.abs(ref))
    wrong = (codes.astype(np.float32) - z16.astype(np.float32).repeat(128, axis=1)) * \
        s16.astype(np.float32).repeat(128, axis=1)
    assert np.max(np.abs(O.matvec_f16w(wrong.astype(np.float16), x) - ref)) > 1e-3
