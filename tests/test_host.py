"""Host-side pieces (CPU only): the library's INT4 quantizer against the oracle,
the weight layout contract, and the C ABI surface (symbols, error paths that
need no GPU)."""
import ctypes as C
import glob
import os
import re

import numpy as np
import pytest

import oracle as O
from ironmill_amd import _lib, quant

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("n,k,scale,seed", [(64, 256, 0.02, 0), (33, 1024, 1.0, 1), (128, 128, 1e-3, 2)])
def test_quantizer_bit_exact_with_oracle(n, k, scale, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * scale).astype(np.float32)
    q = quant.quantize_int4(w)
    packed, sc, zp = O.quantize_tensor_int4(w, 128)
    assert np.array_equal(q.data.reshape(-1), packed)
    assert np.array_equal(q.scales_f32.view(np.uint32), sc.view(np.uint32))
    assert np.array_equal(q.zeros_f32.view(np.uint32), zp.view(np.uint32))
    # GPU upload copies are the f32 params rounded to f16 (convert_params_to_f16)
    assert np.array_equal(q.scales.view(np.uint16), O.convert_params_to_f16(sc).view(np.uint16))
    assert np.array_equal(q.zeros.view(np.uint16), O.convert_params_to_f16(zp).view(np.uint16))


def test_quantizer_edge_groups():
    k = 128
    rows = [
        np.full(k, 0.25, np.float32),                        # degenerate (all equal)
        np.linspace(1.0, 2.0, k, dtype=np.float32),          # all-positive group: negative zp
        np.linspace(-2.0, -1.0, k, dtype=np.float32),        # all-negative group
        np.where(np.arange(k) % 2 == 0, 0.5, -0.5).astype(np.float32),  # exact ties
        np.concatenate([np.float32([np.inf, -np.inf, np.nan]), np.linspace(-1, 1, k - 3, dtype=np.float32)]),
    ]
    w = np.stack(rows)
    q = quant.quantize_int4(w)
    packed, sc, zp = O.quantize_tensor_int4(w, 128)
    assert np.array_equal(q.data.reshape(-1), packed)
    assert np.array_equal(q.scales_f32.view(np.uint32), sc.view(np.uint32))
    assert np.array_equal(q.zeros_f32.view(np.uint32), zp.view(np.uint32))


def test_awq_scales_fold_into_weights():
    """quantized.rs:936-950: W * s is quantized and s travels as f16; (x / s) . (W s) ~ x . W."""
    rng = np.random.default_rng(4)
    n, k = 16, 512
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    s = rng.uniform(0.5, 2.0, k).astype(np.float32)
    q = quant.quantize_int4(w, awq_scales=s)
    packed, sc, zp = O.quantize_tensor_int4((w * s[None, :]).astype(np.float32), 128)
    assert np.array_equal(q.data.reshape(-1), packed)
    assert np.array_equal(q.awq.view(np.uint16), s.astype(np.float16).view(np.uint16))
    x = rng.standard_normal((1, k)).astype(np.float16)
    wdq = O.dequant_affine_int4(packed, sc, zp, n, k)
    y = O.matvec_f16w(wdq, x, q.awq)[0]
    exact = w.astype(np.float64) @ x[0].astype(np.float64)
    assert np.linalg.norm(y - exact) / np.linalg.norm(exact) < 0.2  # INT4 g128 quantisation noise (~12 %)


def test_layout_contract():
    """data [n, k/2] with element 2i in the low nibble; scales/zeros [n, k/128]."""
    w = np.zeros((2, 256), np.float32)
    w[1, 0] = -1.0   # min of group 0 of row 1 -> code 0
    w[1, 3] = 1.0    # max -> the top codes
    q = quant.quantize_int4(w)
    assert q.data.shape == (2, 128) and q.scales.shape == (2, 2) and q.zeros.shape == (2, 2)
    zp = int(q.zeros_f32[1, 0])
    assert q.scales_f32[1, 0] == np.float32(2.0) / np.float32(15.0) and zp == 7
    assert q.data[1, 0] & 0x0F == 0          # element 0 (the min): low nibble of byte 0
    assert q.data[1, 0] >> 4 == zp           # element 1 (0.0) sits at the zero point
    assert q.data[1, 1] & 0x0F == zp         # element 2 (0.0): low nibble of byte 1
    assert q.data[1, 1] >> 4 >= 14           # element 3 (the max): high nibble of byte 1


def _header_functions():
    """Every function the headers under include/ declare."""
    names = set()
    for h in sorted(glob.glob(os.path.join(REPO, "include", "*.h"))):
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names.update(re.findall(r"\b(imh_[a-z0-9_]+)\s*\(", src))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    names = _header_functions()
    assert len(names) >= 30
    lib = C.CDLL(_lib.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(_lib.SIGNATURES) == names  # the Python binding declares exactly these


def test_error_paths_without_gpu():
    L = _lib.lib
    assert L.imh_tq_cache_sizes(1, 8, 128, 64, None, None) == _lib.IMH_EINVAL
    assert b"NULL" in L.imh_last_error()
    cb, sb = C.c_size_t(), C.c_size_t()
    assert L.imh_tq_cache_sizes(2, 8, 128, 1000, C.byref(cb), C.byref(sb)) == 0
    assert cb.value == 2 * 8 * 1000 * 128 and sb.value == 2 * 8 * 1000 * 4
    assert L.imh_device_open(0, None) == _lib.IMH_EINVAL
    assert L.imh_encode_affine_projection_int4(None, None, 1, None, None) == _lib.IMH_EINVAL
    assert b"NULL" in L.imh_last_error()
    n = C.c_int(-1)
    L.imh_device_count(C.byref(n))  # no GPU here: an error code or 0, never a crash
    assert n.value >= 0


def test_rope_cache_is_bit_exact_with_oracle():
    """imh_rope_cache_fill runs on the host: every f16 entry equals the oracle's."""
    import oracle as O
    from ironmill_amd import ops
    for hd, mp, theta, rd in ((128, 4096, 1e6, 0), (128, 300, 1e4, 32), (64, 100, 5e5, 0)):
        c, s = ops.rope_cache(hd, mp, theta, rd)
        c2, s2 = O.rope_cache(hd, mp, theta, rd or None)
        assert np.array_equal(c.view(np.uint16), c2.view(np.uint16))
        assert np.array_equal(s.view(np.uint16), s2.view(np.uint16))


def test_kv_positions_sliding_window_semantics():
    """imh_kv_positions_for (attention.rs:141-163) against what a ring of W slots must show:
    decoding one token at a time, writing token p at write_pos, the slots [0, attn_len) hold
    exactly the last min(p + 1, W) tokens; full-attention layers keep the linear positions."""
    from ironmill_amd import ops
    for W in (1, 3, 8):
        ring = [None] * W
        for p in range(3 * W + 2):
            kp = ops.kv_positions(p, 1, W, 1000)
            assert kp["stride"] == W
            ring[kp["write_pos"]] = p
            visible = sorted(ring[:kp["attn_len"]])
            assert visible == list(range(max(0, p + 1 - W), p + 1)), (W, p, visible)
    kp = ops.kv_positions(17, 4, 0, 64)
    assert kp == {"stride": 64, "write_pos": 17, "attn_base": 17, "attn_len": 21}
    # a prefill chunk inside a window that has not wrapped: the linear positions
    assert ops.kv_positions(2, 3, 8, 64) == {"stride": 8, "write_pos": 2, "attn_base": 2, "attn_len": 5}
    # a chunk that reaches past the window: the attention base clamps so base + T <= W
    kp = ops.kv_positions(7, 3, 8, 64)
    assert kp["write_pos"] == 7 and kp["attn_base"] == 5 and kp["attn_len"] == 8


def test_kv_positions_errors():
    from ironmill_amd import IronmillError, ops
    with pytest.raises(IronmillError, match="exceeds max_seq_len"):
        ops.kv_positions(62, 3, 0, 64)
    with pytest.raises(IronmillError, match="token_count"):
        ops.kv_positions(0, 0, 0, 64)
    with pytest.raises(IronmillError, match="token_count"):
        ops.kv_positions(0, 5, 4, 64)
