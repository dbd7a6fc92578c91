"""ctypes binding of the C oracle (``oracle/_build/liboracle.so``).

Test infrastructure only (see ``oracle/__init__.py``).  Every wrapper takes and
returns numpy arrays; f16 travels as ``np.float16`` (bit patterns are shared
with the C side as uint16).  The composition helpers at the bottom (gate+up,
activations) restate ``affine_fused.metal:89-107`` / ``activation.metal:15-31``
on top of the C matvec.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc; no GPU needed)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
SZ = C.c_size_t


def _declare(L):
    sig = {
        "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_f16_array": (None, [P, P, SZ]),
        "orc_quantize_affine": (None, [P, SZ, C.c_float, P, P, P]),
        "orc_pack_int4": (None, [P, SZ, P]),
        "orc_unpack_int4": (None, [P, SZ, P]),
        "orc_pack_int4_u32": (None, [P, SZ, P]),
        "orc_quantize_tensor_int4": (None, [P, SZ, SZ, SZ, P, P, P]),
        "orc_convert_params_to_f16": (None, [P, SZ, P]),
        "orc_dequant_affine_int4": (None, [P, P, P, SZ, SZ, SZ, P]),
        "orc_dequant_affine_int4_f16params": (None, [P, P, P, SZ, SZ, SZ, P]),
        "orc_matvec_f16w": (None, [P, P, P, SZ, SZ, SZ, P, C.c_int]),
        "orc_silu": (C.c_float, [C.c_float]),
        "orc_gelu_tanh": (C.c_float, [C.c_float]),
        "orc_fused_residual_norm_matvec": (None, [P, P, P, P, C.c_float, P, SZ, SZ, SZ, P, P, P]),
        "orc_lloyd_max_gaussian": (None, [C.c_int, C.c_int, P, P]),
        "orc_normal_quantile": (C.c_double, [C.c_double]),
        "orc_erf": (C.c_double, [C.c_double]),
        "orc_chacha_block": (None, [P, C.c_int, P]),
        "orc_rotation_signs": (None, [C.c_int, C.c_uint64, P]),
        "orc_qjl_matrix": (None, [C.c_int, C.c_uint64, P]),
        "orc_hadamard_rotate": (None, [P, P, C.c_int]),
        "orc_tq_quantize_vector": (None, [P, C.c_int, C.c_int, P, P, P, C.c_int, P, P, P, P]),
        "orc_tq_cache_write": (None, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P,
                                      C.c_int, P, P, P, C.c_int, P, P, P, P]),
        "orc_fp16_attention": (None, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_int, P, C.c_float, P, P, P, C.c_int]),
        "orc_tq_attention": (None, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P,
                                    C.c_float, P, P, P, P, P, P, P, P, P, P, C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- f16

def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out.view(np.float16)


# ---------------------------------------------------------------- INT4

def quantize_affine(values, qmax=15.0):
    v = _c(values, np.float32)
    q = np.zeros(v.size, np.uint8)
    s = C.c_float()
    z = C.c_float()
    lib().orc_quantize_affine(_p(v), v.size, qmax, _p(q), C.byref(s), C.byref(z))
    return q, np.float32(s.value), np.float32(z.value)


def pack_int4(values) -> np.ndarray:
    v = _c(values, np.uint8)
    out = np.zeros((v.size + 1) // 2, np.uint8)
    lib().orc_pack_int4(_p(v), v.size, _p(out))
    return out


def unpack_int4(packed, count) -> np.ndarray:
    p = _c(packed, np.uint8)
    out = np.zeros(count, np.uint8)
    lib().orc_unpack_int4(_p(p), count, _p(out))
    return out


def pack_int4_u32(values) -> np.ndarray:
    v = _c(values, np.uint8)
    out = np.zeros((v.size + 7) // 8, np.uint32)
    lib().orc_pack_int4_u32(_p(v), v.size, _p(out))
    return out


def quantize_tensor_int4(w, gs=128):
    """quantized.rs:408-465 -> (packed u8 [ceil(n*k/2)], scales f32 [n,G], zeros f32 [n,G])."""
    w = _c(w, np.float32)
    rows, k = w.shape
    ng = -(-k // gs)
    packed = np.zeros((rows * k + 1) // 2, np.uint8)
    scales = np.zeros((rows, ng), np.float32)
    zeros = np.zeros((rows, ng), np.float32)
    lib().orc_quantize_tensor_int4(_p(w), rows, k, gs, _p(packed), _p(scales), _p(zeros))
    return packed, scales, zeros


def convert_params_to_f16(p) -> np.ndarray:
    p = _c(p, np.float32)
    out = np.zeros(p.shape, np.uint16)
    lib().orc_convert_params_to_f16(_p(p), p.size, _p(out))
    return out.view(np.float16)


def dequant_affine_int4(packed, scales, zeros, n, k, gs=128) -> np.ndarray:
    """dequant.rs:85-180 (group branch), f32 params -> dense f16 [n,k]."""
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.float32)
    zeros = _c(zeros, np.float32)
    out = np.zeros((n, k), np.uint16)
    lib().orc_dequant_affine_int4(_p(packed), _p(scales), _p(zeros), n, k, gs, _p(out))
    return out.view(np.float16)


def dequant_affine_int4_f16params(packed, scales16, zeros16, n, k, gs=128) -> np.ndarray:
    packed = _c(packed, np.uint8)
    s = _c(scales16, np.float16).view(np.uint16)
    z = _c(zeros16, np.float16).view(np.uint16)
    out = np.zeros((n, k), np.uint16)
    lib().orc_dequant_affine_int4_f16params(_p(packed), _p(s), _p(z), n, k, gs, _p(out))
    return out.view(np.float16)


def matvec_f16w(w16, x16, awq16=None, nthreads=1) -> np.ndarray:
    """y[b, n] = sum_k (x[b,k] (/ awq[k])) * W[n,k], f32 accumulate -> f32 [B, N]."""
    w = _c(w16, np.float16).view(np.uint16)
    x = _c(x16, np.float16).view(np.uint16)
    if x.ndim == 1:
        x = x[None, :]
    a = None if awq16 is None else _c(awq16, np.float16).view(np.uint16)
    n, k = w.shape
    b = x.shape[0]
    y = np.zeros((b, n), np.float32)
    lib().orc_matvec_f16w(_p(w), _p(x), _p(a), b, n, k, _p(y), nthreads)
    return y


def silu(g):
    g = np.asarray(g, np.float32)
    return np.vectorize(lambda v: lib().orc_silu(float(v)), otypes=[np.float32])(g)


def gelu_tanh(g):
    g = np.asarray(g, np.float32)
    return np.vectorize(lambda v: lib().orc_gelu_tanh(float(v)), otypes=[np.float32])(g)


def gate_up_act(w_gate16, w_up16, x16, awq16=None, act="silu"):
    """affine_fused.metal:89-107: out = f16(act(gate) * up), gate/up in f32."""
    g = matvec_f16w(w_gate16, x16, awq16)
    u = matvec_f16w(w_up16, x16, awq16)
    a = silu(g) if act == "silu" else gelu_tanh(g)
    return (a * u).astype(np.float32)


def fused_residual_norm_matvec(a16, b16, gamma16, w16, eps, awq16=None):
    a = _c(a16, np.float16).view(np.uint16)
    b = _c(b16, np.float16).view(np.uint16)
    if a.ndim == 1:
        a, b = a[None, :], b[None, :]
    g = _c(gamma16, np.float16).view(np.uint16)
    aw = None if awq16 is None else _c(awq16, np.float16).view(np.uint16)
    w = _c(w16, np.float16).view(np.uint16)
    n, k = w.shape
    m = a.shape[0]
    y = np.zeros((m, n), np.float32)
    res = np.zeros((m, k), np.uint16)
    nrm = np.zeros((m, k), np.uint16)
    lib().orc_fused_residual_norm_matvec(_p(a), _p(b), _p(g), _p(aw), eps, _p(w), m, n, k,
                                         _p(y), _p(res), _p(nrm))
    return y, res.view(np.float16), nrm.view(np.float16)


# ---------------------------------------------------------------- TurboQuant

def lloyd_max_gaussian(dim, bits):
    n = 1 << bits
    lv = np.zeros(n, np.float32)
    bd = np.zeros(max(n - 1, 1), np.float32)
    lib().orc_lloyd_max_gaussian(dim, bits, _p(lv), _p(bd))
    return lv, bd[: n - 1]


def normal_quantile(p):
    return lib().orc_normal_quantile(float(p))


def erf(x):
    return lib().orc_erf(float(x))


def chacha_block(words16, rounds=20):
    w = _c(words16, np.uint32)
    out = np.zeros(16, np.uint32)
    lib().orc_chacha_block(_p(w), rounds, _p(out))
    return out


def rotation_signs(dim, seed):
    s = np.zeros(dim, np.float32)
    lib().orc_rotation_signs(dim, seed, _p(s))
    return s


def qjl_matrix(dim, seed):
    s = np.zeros((dim, dim), np.float32)
    lib().orc_qjl_matrix(dim, seed, _p(s))
    return s


def hadamard_rotate(x, signs):
    x = _c(x, np.float32).copy()
    s = _c(signs, np.float32)
    lib().orc_hadamard_rotate(_p(x), _p(s), x.size)
    return x


class TQTables:
    """Host copy of the TurboQuant tables (metal/turboquant/mod.rs:221-287):
    K uses the (n_bits-1)-bit codebook, V the n_bits codebook, QJL seed+1."""

    def __init__(self, head_dim=128, n_bits=8, seed=42):
        self.head_dim, self.n_bits, self.seed = head_dim, n_bits, seed
        self.signs = rotation_signs(head_dim, seed)
        self.k_codebook, self.k_bounds = lloyd_max_gaussian(head_dim, n_bits - 1)
        self.v_codebook, self.v_bounds = lloyd_max_gaussian(head_dim, n_bits)
        self.qjl = qjl_matrix(head_dim, seed + 1)


def tq_quantize_vector(x16, tables: TQTables, is_k: bool):
    x = _c(x16, np.float16).view(np.uint16)
    d = x.size
    codes = np.zeros(d, np.uint8)
    sc = C.c_float()
    rn = C.c_float()
    cb = tables.k_codebook if is_k else tables.v_codebook
    bd = tables.k_bounds if is_k else tables.v_bounds
    lib().orc_tq_quantize_vector(_p(x), d, int(is_k), _p(tables.signs), _p(cb), _p(bd), cb.size,
                                 _p(tables.qjl), _p(codes), C.byref(sc), C.byref(rn))
    return codes, np.float32(sc.value), np.float32(rn.value)


def tq_cache_write(kv16, tables: TQTables, is_k, max_seq, base_pos=0, positions=None,
                   cache=None, scales=None, r_norms=None):
    """kv16: [B, T, nkv, d] -> (cache [B,nkv,max_seq,d] u8, scales, r_norms [B,nkv,max_seq])."""
    kv = _c(kv16, np.float16).view(np.uint16)
    b, t, nkv, d = kv.shape
    if cache is None:
        cache = np.zeros((b, nkv, max_seq, d), np.uint8)
        scales = np.zeros((b, nkv, max_seq), np.float32)
        r_norms = np.zeros((b, nkv, max_seq), np.float32)
    pos = None if positions is None else _c(positions, np.int32)
    cb = tables.k_codebook if is_k else tables.v_codebook
    bd = tables.k_bounds if is_k else tables.v_bounds
    lib().orc_tq_cache_write(_p(kv), b, t, nkv, d, max_seq, base_pos, _p(pos), int(is_k),
                             _p(tables.signs), _p(cb), _p(bd), cb.size, _p(tables.qjl),
                             _p(cache), _p(scales), _p(r_norms))
    return cache, scales, r_norms


def tq_attention(q16, tables: TQTables, k_cache, v_cache, k_scales, v_scales, k_r_norms,
                 seq_len, attn_scale, seq_lens=None, nthreads=1):
    """q16: [B, nh, d]; caches as from tq_cache_write -> f32 [B, nh, d]."""
    q = _c(q16, np.float16).view(np.uint16)
    b, nh, d = q.shape
    nkv, max_seq = k_cache.shape[1], k_cache.shape[2]
    out = np.zeros((b, nh, d), np.float32)
    sl = None if seq_lens is None else _c(seq_lens, np.int32)
    lib().orc_tq_attention(_p(q), b, nh, nkv, d, max_seq, seq_len, _p(sl), attn_scale,
                           _p(tables.signs), _p(tables.k_codebook), _p(tables.v_codebook),
                           _p(tables.qjl), _p(_c(k_cache, np.uint8)), _p(_c(v_cache, np.uint8)),
                           _p(_c(k_scales, np.float32)), _p(_c(v_scales, np.float32)),
                           _p(_c(k_r_norms, np.float32)), _p(out), nthreads)
    return out


def fp16_attention(q16, k_cache16, v_cache16, seq_len, attn_scale, seq_lens=None, nthreads=1):
    """q16: [B, nh, d] (one token) or [B, T, nh, d]; caches [B, nkv, max_seq, d]
    f16 -> f32 of q's shape.  Token t attends to p < seq_len - T + t + 1."""
    q = _c(q16, np.float16).view(np.uint16)
    squeeze = q.ndim == 3
    if squeeze:
        q = q[:, None]
    k = _c(k_cache16, np.float16).view(np.uint16)
    v = _c(v_cache16, np.float16).view(np.uint16)
    b, t, nh, d = q.shape
    nkv, max_seq = k.shape[1], k.shape[2]
    out = np.zeros((b, t, nh, d), np.float32)
    sl = None if seq_lens is None else _c(seq_lens, np.int32)
    lib().orc_fp16_attention(_p(_c(q, np.uint16)), b, t, nh, nkv, d, max_seq, seq_len, _p(sl), attn_scale,
                             _p(k), _p(v), _p(out), nthreads)
    return out[:, 0] if squeeze else out
