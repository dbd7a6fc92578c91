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
        "orc_quantize_tensor_int8": (None, [P, SZ, SZ, SZ, P, P, P]),
        "orc_dequant_affine_int8": (None, [P, P, P, SZ, SZ, SZ, P]),
        "orc_quantize_input_q8": (None, [P, SZ, SZ, SZ, P, P]),
        "orc_matvec_int4xq8": (None, [P, P, P, P, P, SZ, SZ, SZ, SZ, P]),
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
        "orc_pcg32_advance": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "orc_pcg32_xsh_rr": (C.c_uint32, [C.c_uint64]),
        "orc_stdrng_stream": (None, [P, C.c_uint64, C.c_int, P]),
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


def quantize_tensor_int8(w, gs=128):
    """quantized.rs:852-901 -> (codes u8 [rows, k], scales f32 [rows, G], zeros f32 [rows, G])."""
    w = _c(w, np.float32)
    rows, k = w.shape
    ng = -(-k // gs)
    codes = np.zeros((rows, k), np.uint8)
    scales = np.zeros((rows, ng), np.float32)
    zeros = np.zeros((rows, ng), np.float32)
    lib().orc_quantize_tensor_int8(_p(w), rows, k, gs, _p(codes), _p(scales), _p(zeros))
    return codes, scales, zeros


def dequant_affine_int8(codes, scales, zeros, n, k, gs=128) -> np.ndarray:
    """dequant.rs:122-142 for 8-bit codes, f32 params -> dense f16 [n, k]."""
    out = np.zeros((n, k), np.uint16)
    lib().orc_dequant_affine_int8(_p(_c(codes, np.uint8)), _p(_c(scales, np.float32)), _p(_c(zeros, np.float32)),
                                  n, k, gs, _p(out))
    return out.view(np.float16)


def quantize_input_q8(x16, gs=128):
    """quantize.metal:21-52 per row -> (q8 int8 [rows, k], scales f32 [rows, k/gs])."""
    x = _c(x16, np.float16).view(np.uint16)
    if x.ndim == 1:
        x = x[None, :]
    rows, k = x.shape
    q8 = np.zeros((rows, k), np.int8)
    sc = np.zeros((rows, k // gs), np.float32)
    lib().orc_quantize_input_q8(_p(x), rows, k, gs, _p(q8), _p(sc))
    return q8, sc


def matvec_int4xq8(q8, q8_scales, packed, scales16, zeros16, n, k, gs=128) -> np.ndarray:
    """affine_fused.metal:115-176 restated exactly (integer group sums) -> f64 [rows, n]."""
    q8 = _c(q8, np.int8)
    rows = q8.shape[0]
    y = np.zeros((rows, n), np.float64)
    lib().orc_matvec_int4xq8(_p(q8), _p(_c(q8_scales, np.float32)), _p(_c(packed, np.uint8)),
                             _p(_c(scales16, np.float16).view(np.uint16)), _p(_c(zeros16, np.float16).view(np.uint16)),
                             rows, n, k, gs, _p(y))
    return y


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


def bf16_round(x) -> np.ndarray:
    """IEEE f32 -> bfloat16 with round-to-nearest-even, as uint16 bit patterns (finite inputs)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_round(x) -> np.ndarray:
    """OCP FP8 E4M3 (bias 7, 3 mantissa bits, subnormal quantum 2^-9, largest finite 448):
    f32 -> the nearest e4m3 value (ties to even), saturating at +-448, returned as f32."""
    v = np.clip(np.asarray(x, np.float32).astype(np.float64), -448.0, 448.0)
    _, e = np.frexp(v)                        # v = m 2^e, 0.5 <= |m| < 1
    q = np.exp2(np.maximum(e - 4, -9))        # spacing of the binade (subnormal below 2^-6)
    return (np.rint(v / q) * q).astype(np.float32)


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


def pcg32_advance(state, inc):
    return int(lib().orc_pcg32_advance(state & (2 ** 64 - 1), inc & (2 ** 64 - 1)))


def pcg32_xsh_rr(state):
    return int(lib().orc_pcg32_xsh_rr(state & (2 ** 64 - 1)))


def stdrng_stream(n, seed=0, key=None):
    """n u64 draws of StdRng: keyed by the 8 words `key`, else seed_from_u64(seed)."""
    out = np.zeros(n, np.uint64)
    k = None if key is None else _c(key, np.uint32)
    lib().orc_stdrng_stream(_p(k), seed, n, _p(out))
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


# ------------------------------------------------------------ decode-step glue
# numpy restatements in f64 arithmetic with f16 storage at the points where the
# kernels store f16.

def _f64(x16):
    return np.asarray(x16, np.float16).astype(np.float64)


def rms_norm(x16, w16, eps):
    """rms_norm (normalization.metal:19-57): f16(x * 1/sqrt(mean(x^2)+eps) * w) per row."""
    x = _f64(x16)
    inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return (x * inv * _f64(w16)).astype(np.float16)


def fused_residual_rms_norm(a16, b16, w16, eps):
    """fused_residual_rms_norm (fused_residual_norm.metal:33-75) -> (normed, residual)."""
    x = _f64(a16) + _f64(b16)
    inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return (x * inv * _f64(w16)).astype(np.float16), x.astype(np.float16)


def residual_add(a16, b16):
    return (_f64(a16) + _f64(b16)).astype(np.float16)


def fused_embedding_norm(ids, table16, w16, eps, embed_scale=1.0):
    """fused_embedding_norm (fused_embedding_norm.metal:29-73) -> (normed, raw); ids >= vocab give 0."""
    ids = np.asarray(ids, np.int64)
    vocab = table16.shape[0]
    valid = (ids >= 0) & (ids < vocab)
    x = np.where(valid[:, None], _f64(table16[np.where(valid, ids, 0)]) * np.float64(np.float32(embed_scale)), 0.0)
    inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return (x * inv * _f64(w16)).astype(np.float16), x.astype(np.float16)


def rope_cache(head_dim, max_pos, theta, rotary_dim=None):
    """precompute_rope_cache (ironmill-core/src/rope.rs:22-50): f16 cos/sin [max_pos, head_dim/2],
    f64 angles rounded once to f16 (numpy's double -> half cast rounds to nearest even)."""
    half = head_dim // 2
    rd = rotary_dim or head_dim
    i = np.arange(half, dtype=np.float64)
    freq = 1.0 / np.power(np.float64(theta), 2.0 * i / rd)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * freq[None, :]
    cos, sin = np.cos(ang), np.sin(ang)
    cos[:, rd // 2:] = 1.0
    sin[:, rd // 2:] = 0.0
    return cos.astype(np.float16), sin.astype(np.float16)


def qk_norm_rope(x16, norm_w16, cos16, sin16, pos, eps, rotary_dim=None):
    """One tensor of encode_qk_norm_and_rope (attention.rs:26-92) for rows x16 [..., heads, hd]
    at integer positions pos (broadcast over heads).  With norm_w16: fused_qk_norm_rope
    (fused_qk_norm_rope.metal:43-124), pairs (d, d + rotary/2); without: rope.metal, pairs
    (d, d + hd/2)."""
    x = _f64(x16)
    hd = x.shape[-1]
    pos = np.asarray(pos, np.int64)
    c = _f64(cos16)[pos][..., None, :]   # [..., 1, hd/2]
    s = _f64(sin16)[pos][..., None, :]
    out = x.copy()
    if norm_w16 is not None:
        rd = rotary_dim or hd
        hr = rd // 2
        inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
        y = x * inv * _f64(norm_w16)
        lo, hi = y[..., :hr], y[..., hr:rd]
        out[..., :hr] = lo * c[..., :hr] - hi * s[..., :hr]
        out[..., hr:rd] = lo * s[..., :hr] + hi * c[..., :hr]
        out[..., rd:] = y[..., rd:]
    else:
        h = hd // 2
        lo, hi = x[..., :h], x[..., h:]
        out[..., :h] = lo * c - hi * s
        out[..., h:] = lo * s + hi * c
    return out.astype(np.float16)


class DecoderReference:
    """The decode step of run_pipeline_inner (metal/pipeline.rs:424-1172, token_count 1) restated
    on the CPU over the dequantize-then-compute ops: every projection uses the f16 dense weight
    of dequant_affine (core/dequant.rs:85-180) with an f32 accumulator; activations are stored
    as f16 at the same points as the GPU buffers (norm_out, q/k/v, attn_out, ffn_down, residual,
    hidden); attention runs on the cache as written (FP16 rows, or TurboQuant codes from
    tq_cache_write).

    layers: list of dicts with input_norm, post_attn_norm, q_norm, k_norm (f16 arrays or None)
    and q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj (objects with data,
    scales_f32, zeros_f32, awq, n, k; for weights="exact" also scales / zeros f16).

    Variants for sensitivity studies (the default is the reference's CPU path):
      weights="exact": the GPU upload's weight semantics instead of the CPU dequant --
        w = (q - z16) * s16 with the f16 scales and zero-points (metal/weights.rs:1064-1103,
        core/dequant.rs:305-345), exact in f32, not rounded to f16;
      acc="f64": projections accumulate in float64 (numpy) instead of a sequential f32 sum,
        which changes only the rounding of the f32 result (weights="exact" only).
    tables: TQTables to use instead of TQTables(head_dim, 8, tq_seed).
    window_sizes: per-layer sliding windows (0 = full attention): a windowed layer attends, at
      position p, to the positions [max(0, p + 1 - W), p] -- the definition the reference's ring
      buffer of W slots implements (attention.rs:141-163); this cache stays linear."""

    def __init__(self, cfg: dict, layers, embedding16, final_norm16, lm_head, kv_cache="turboquant",
                 tq_seed=42, weights="f16", acc="f32", tables=None, window_sizes=None):
        if weights not in ("f16", "exact") or acc not in ("f32", "f64"):
            raise ValueError("weights must be 'f16' or 'exact', acc 'f32' or 'f64'")
        if weights == "f16" and acc != "f32":
            raise ValueError("the f16-weight path accumulates in f32 (the reference's CPU path)")
        self.exact = weights == "exact"
        self.acc = np.float64 if acc == "f64" else np.float32
        self.cfg = dict(cfg)
        c = self.cfg
        self.B = c["batch"]
        self.nh, self.nkv, self.hd = c["num_heads"], c["num_kv_heads"], c["head_dim"]
        self.eps = c.get("rms_eps", 1e-6)
        self.scale = c.get("attn_scale") or 1.0 / np.sqrt(self.hd)
        self.max_seq = c["max_seq_len"]
        self.cos, self.sin = rope_cache(self.hd, self.max_seq, c.get("rope_theta", 1e6), c.get("rotary_dim") or None)
        self.kv = kv_cache
        self.emb = np.asarray(embedding16, np.float16)
        self.final_norm = final_norm16
        self.layers = []
        memo = {}   # a weight object shared by several layers is dequantized once
        for L in layers:
            d = dict(L)
            for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
                if id(L[name]) not in memo:
                    memo[id(L[name])] = self._dense(L[name])
                d[name] = memo[id(L[name])]
            self.layers.append(d)
        self.lm = self._dense(lm_head)
        shp = (self.B, self.nkv, self.max_seq)
        if kv_cache == "turboquant":
            self.tables = tables if tables is not None else TQTables(self.hd, 8, tq_seed)
            self.caches = [dict(k_codes=np.zeros(shp + (self.hd,), np.uint8),
                                v_codes=np.zeros(shp + (self.hd,), np.uint8),
                                k_scales=np.zeros(shp, np.float32), v_scales=np.zeros(shp, np.float32),
                                k_r_norms=np.zeros(shp, np.float32)) for _ in layers]
        else:
            self.caches = [dict(k=np.zeros(shp + (self.hd,), np.float16), v=np.zeros(shp + (self.hd,), np.float16))
                           for _ in layers]
        self.positions = np.zeros(self.B, np.int32)
        self.windows = list(window_sizes) if window_sizes is not None else [0] * len(layers)

    def _dense(self, w):
        if not self.exact:
            return (dequant_affine_int4(w.data, w.scales_f32, w.zeros_f32, w.n, w.k), w.awq)
        q = unpack_int4(np.asarray(w.data).reshape(-1), w.n * w.k).reshape(w.n, w.k // 128, 128)
        z = np.asarray(w.zeros, np.float16).astype(np.float32)[:, :, None]
        s = np.asarray(w.scales, np.float16).astype(np.float32)[:, :, None]
        return (((q.astype(np.float32) - z) * s).reshape(w.n, w.k).astype(self.acc), w.awq)

    def _act(self, x16, awq):
        x = np.asarray(x16, np.float16).astype(np.float32)
        if awq is not None:
            x = x / np.asarray(awq, np.float16).astype(np.float32)
        return x

    def _matvec(self, w, x16):
        """f32 [B, N] of one projection (x16 [B, K] f16)."""
        dense, awq = w
        if not self.exact:
            return matvec_f16w(dense, x16, awq, nthreads=8)
        return (self._act(x16, awq).astype(self.acc) @ dense.T).astype(np.float32)

    def _proj(self, w, x16):
        return self._matvec(w, x16).astype(np.float16)

    def _gate_up_act(self, g_w, u_w, x16, act):
        if not self.exact:
            return gate_up_act(g_w[0], u_w[0], x16, g_w[1], act=act)
        g = self._matvec((g_w[0], g_w[1]), x16)
        u = self._matvec((u_w[0], g_w[1]), x16)
        a = g / (np.float32(1.0) + np.exp(-g)) if act == "silu" else gelu_tanh(g)
        return (a * u).astype(np.float32)

    def _resnorm_matvec(self, a16, b16, gamma16, w, eps):
        """fused_residual_norm_matvec (superblock_fused_norm.metal:37-124) -> (y, residual, normed)."""
        if not self.exact:
            return fused_residual_norm_matvec(a16, b16, gamma16, w[0], eps, w[1])
        r = np.asarray(a16, np.float16).astype(np.float32) + np.asarray(b16, np.float16).astype(np.float32)
        g = np.asarray(gamma16, np.float16).astype(np.float32)
        rms_inv = (1.0 / np.sqrt((r.astype(np.float64) ** 2).mean(axis=-1, keepdims=True) + eps)).astype(np.float32)
        x = r * g
        if w[1] is not None:
            x = x / np.asarray(w[1], np.float16).astype(np.float32)
        y = (x.astype(self.acc) @ w[0].T).astype(np.float32) * rms_inv
        return y, r.astype(np.float16), (r * rms_inv * g).astype(np.float16)

    def _write_cache(self, l, k16, v16):
        cache, pos = self.caches[l], self.positions
        if self.kv == "turboquant":
            for x, is_k, cn, sn in ((k16, True, "k_codes", "k_scales"), (v16, False, "v_codes", "v_scales")):
                codes, sc, rn = tq_cache_write(x[:, None], self.tables, is_k, self.max_seq, positions=pos)
                for b in range(self.B):
                    p = pos[b] % self.max_seq
                    cache[cn][b, :, p] = codes[b, :, p]
                    cache[sn][b, :, p] = sc[b, :, p]
                    if is_k:
                        cache["k_r_norms"][b, :, p] = rn[b, :, p]
        else:
            for b in range(self.B):
                p = pos[b] % self.max_seq
                cache["k"][b, :, p] = k16[b]
                cache["v"][b, :, p] = v16[b]

    def _attend(self, l, q16):
        cache = self.caches[l]
        W = self.windows[l]
        if W:   # the last W positions of each sequence
            rows = []
            for b in range(self.B):
                e = int(min(self.positions[b] + 1, self.max_seq))
                s0 = max(0, e - W)
                sl = {k: v[b:b + 1, :, s0:e] for k, v in cache.items()}
                if self.kv == "turboquant":
                    o = tq_attention(q16[b:b + 1], self.tables, sl["k_codes"], sl["v_codes"], sl["k_scales"],
                                     sl["v_scales"], sl["k_r_norms"], e - s0, self.scale, nthreads=8)
                else:
                    o = fp16_attention(q16[b:b + 1], sl["k"], sl["v"], e - s0, self.scale, nthreads=8)
                rows.append(o)
            return np.concatenate(rows, axis=0).astype(np.float16)
        lens = np.minimum(self.positions + 1, self.max_seq).astype(np.int32)
        if self.kv == "turboquant":
            out = tq_attention(q16, self.tables, cache["k_codes"], cache["v_codes"], cache["k_scales"],
                               cache["v_scales"], cache["k_r_norms"], 0, self.scale, seq_lens=lens, nthreads=8)
        else:
            out = fp16_attention(q16, cache["k"], cache["v"], 0, self.scale, seq_lens=lens, nthreads=8)
        return out.astype(np.float16)

    def step(self, token_ids, cache_hook=None):
        """One token per sequence -> f32 logits [B, vocab]; advances the positions.
        cache_hook(layer, cache, positions), if given, runs after each layer's cache write
        (a test may substitute the rows the GPU wrote there)."""
        B, nh, nkv, hd, eps = self.B, self.nh, self.nkv, self.hd, self.eps
        L0 = self.layers[0]
        normed, hidden = fused_embedding_norm(token_ids, self.emb, L0["input_norm"], eps,
                                              self.cfg.get("embed_scale") or 1.0)
        q = None
        for l, L in enumerate(self.layers):
            if q is None:
                q = self._proj(L["q_proj"], normed)
            k = self._proj(L["k_proj"], normed)
            v = self._proj(L["v_proj"], normed)
            pos = self.positions
            rd = self.cfg.get("rotary_dim") or None
            q = qk_norm_rope(q.reshape(B, nh, hd), L.get("q_norm"), self.cos, self.sin, pos, eps, rd)
            k = qk_norm_rope(k.reshape(B, nkv, hd), L.get("k_norm"), self.cos, self.sin, pos, eps, rd)
            self._write_cache(l, k, v.reshape(B, nkv, hd))
            if cache_hook is not None:
                cache_hook(l, self.caches[l], self.positions)
            attn = self._attend(l, q)
            o = self._proj(L["o_proj"], attn.reshape(B, nh * hd))
            normed, residual = fused_residual_rms_norm(hidden, o, L["post_attn_norm"], eps)
            act = self._gate_up_act(L["gate_proj"], L["up_proj"], normed,
                                    "gelu" if self.cfg.get("use_gelu") else "silu").astype(np.float16)
            down = self._proj(L["down_proj"], act)
            if l + 1 < len(self.layers):
                nL = self.layers[l + 1]
                y, hidden, normed = self._resnorm_matvec(residual, down, nL["input_norm"], nL["q_proj"], eps)
                q = y.astype(np.float16)
            else:
                hidden = residual_add(residual, down)
                q = None
        normed = rms_norm(hidden, self.final_norm, eps)
        logits = self._matvec(self.lm, normed)
        self.positions = self.positions + 1
        return logits
