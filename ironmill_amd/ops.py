"""Op tier: the HIP backend's encoders, named after the Metal backend's.

Each function enqueues one op of libironmill_hip on a stream and returns
immediately (``Stream.sync()`` waits), like the ``encode_*`` functions of
ironmill-inference/src/metal/{projection.rs, ops/quantized.rs, ops/fused.rs,
attention.rs} that record into a command encoder.  Errors raise
``IronmillError`` carrying the library's message.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np

from . import _lib
from ._lib import AffineInt4Weight, FusedResidualNormParams, TqKvCache, check, lib
from .quant import QuantizedInt4
from .runtime import Buffer, Device, Stream


def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, Buffer):
        return x.ptr
    return int(x)


class AffineQuantizedWeight:
    """Device copy of an INT4 weight (metal/weights.rs:129-147, upload :1036-1114)."""

    def __init__(self, dev: Device, q: QuantizedInt4):
        self.n, self.k, self.group_size = q.n, q.k, q.group_size
        self.data = dev.upload(q.data)
        self.scales = dev.upload(q.scales)
        self.zeros = dev.upload(q.zeros)
        self.awq_scales = dev.upload(q.awq) if q.awq is not None else None
        self._c = AffineInt4Weight(self.data.ptr, self.scales.ptr, self.zeros.ptr,
                                   self.awq_scales.ptr if self.awq_scales is not None else None,
                                   self.n, self.k, self.group_size)

    @classmethod
    def from_pointers(cls, data, scales, zeros, awq, n, k, group_size=128):
        self = cls.__new__(cls)
        self.n, self.k, self.group_size = n, k, group_size
        self.data, self.scales, self.zeros, self.awq_scales = data, scales, zeros, awq
        self._c = AffineInt4Weight(_ptr(data), _ptr(scales), _ptr(zeros), _ptr(awq), n, k, group_size)
        return self

    @property
    def c(self) -> AffineInt4Weight:
        return self._c


def encode_projection(stream: Stream, x, weight: AffineQuantizedWeight, y, token_count: int):
    """encode_projection -> encode_affine_projection (projection.rs:35-56,227-312)."""
    check(lib.imh_encode_affine_projection_int4(stream.handle, _ptr(x), token_count,
                                                C.byref(weight.c), _ptr(y)))


def encode_batched_affine_matvec_int4(stream: Stream, x, gate: AffineQuantizedWeight, gate_out,
                                      up: AffineQuantizedWeight, up_out, token_count: int = 1):
    """ops/quantized.rs:198-232."""
    check(lib.imh_encode_batched_affine_matvec_int4(stream.handle, _ptr(x), token_count,
                                                    C.byref(gate.c), _ptr(gate_out), C.byref(up.c),
                                                    _ptr(up_out)))


def encode_fused_ffn_gate_up_act_int4(stream: Stream, x, gate: AffineQuantizedWeight,
                                      up: AffineQuantizedWeight, out, token_count: int = 1,
                                      use_gelu: bool = False):
    """ops/quantized.rs:238-270."""
    check(lib.imh_encode_fused_ffn_gate_up_act_int4(stream.handle, _ptr(x), token_count,
                                                    C.byref(gate.c), C.byref(up.c), _ptr(out),
                                                    int(bool(use_gelu))))


def encode_fused_residual_norm_affine_matvec_int4(stream: Stream, a, b, norm_weight, residual_output,
                                                  weight: AffineQuantizedWeight, output,
                                                  normed_output, eps: float, token_count: int = 1):
    """ops/fused.rs:102-129 with FusedResidualNormAffineInt4Params (ops/fused.rs:45-66)."""
    p = FusedResidualNormParams(_ptr(a), _ptr(b), _ptr(norm_weight), _ptr(residual_output),
                                C.pointer(weight.c), _ptr(output), _ptr(normed_output), token_count,
                                eps)
    check(lib.imh_encode_fused_residual_norm_affine_matvec_int4(stream.handle, C.byref(p)))


# ------------------------------------------------------------------ TurboQuant


class TurboQuantModel:
    """MetalTurboQuantModel counterpart (metal/turboquant/mod.rs:51-79,221-287)."""

    def __init__(self, dev: Device, head_dim: int = 128, n_bits: int = 8, rotation_seed: int = 42,
                 host_tables: dict | None = None):
        h = C.c_void_p()
        if host_tables is None:
            check(lib.imh_tq_tables_create(dev.handle, head_dim, n_bits, rotation_seed, C.byref(h)))
        else:
            arrs = [np.ascontiguousarray(host_tables[k], np.float32)
                    for k in ("signs", "k_codebook", "k_bounds", "v_codebook", "v_bounds", "qjl")]
            check(lib.imh_tq_tables_create_from_host(dev.handle, head_dim, n_bits,
                                                     *[a.ctypes.data_as(C.c_void_p) for a in arrs],
                                                     C.byref(h)))
        self._h = h
        self._dev = dev
        self.head_dim, self.n_bits = head_dim, n_bits

    @property
    def handle(self):
        return self._h

    def read(self, which: int) -> np.ndarray:
        n = C.c_size_t()
        check(lib.imh_tq_tables_read(self._h, which, None, 0, C.byref(n)))
        out = np.zeros(n.value, np.float32)
        check(lib.imh_tq_tables_read(self._h, which, out.ctypes.data_as(C.c_void_p), out.size,
                                     C.byref(n)))
        return out

    def tables(self) -> dict:
        names = ["signs", "k_codebook", "k_bounds", "v_codebook", "v_bounds", "qjl"]
        t = {nm: self.read(i) for i, nm in enumerate(names)}
        t["qjl"] = t["qjl"].reshape(self.head_dim, self.head_dim)
        return t

    def close(self):
        if getattr(self, "_h", None):
            lib.imh_tq_tables_free(self._h)
            self._h = None

    def __del__(self):
        self.close()


class TurboQuantKvCache:
    """One layer of MetalKvCache (metal/turboquant/cache.rs:45-96) for `batch` sequences."""

    def __init__(self, dev: Device, batch: int, num_kv_heads: int, head_dim: int, max_seq_len: int):
        codes, scales = C.c_size_t(), C.c_size_t()
        check(lib.imh_tq_cache_sizes(batch, num_kv_heads, head_dim, max_seq_len, C.byref(codes),
                                     C.byref(scales)))
        self.batch, self.num_kv_heads, self.head_dim, self.max_seq_len = (
            batch, num_kv_heads, head_dim, max_seq_len)
        shp = (batch, num_kv_heads, max_seq_len)
        self.k_codes = dev.empty(shp + (head_dim,), np.uint8)
        self.v_codes = dev.empty(shp + (head_dim,), np.uint8)
        self.k_scales = dev.empty(shp, np.float32)
        self.v_scales = dev.empty(shp, np.float32)
        self.k_r_norms = dev.empty(shp, np.float32)
        self._c = TqKvCache(self.k_codes.ptr, self.v_codes.ptr, self.k_scales.ptr, self.v_scales.ptr,
                            self.k_r_norms.ptr, batch, num_kv_heads, head_dim, max_seq_len)

    @property
    def c(self) -> TqKvCache:
        return self._c

    def zero(self, stream: Stream):
        for b in (self.k_codes, self.v_codes, self.k_scales, self.v_scales, self.k_r_norms):
            stream.zero(b)


def encode_turboquant_cache_write(stream: Stream, tq: TurboQuantModel, cache: TurboQuantKvCache,
                                  kv_proj, token_count: int, base_pos: int, is_k: bool,
                                  positions=None):
    """turboquant_cache_write as encoded at attention.rs:344-391."""
    check(lib.imh_encode_turboquant_cache_write(stream.handle, tq.handle, C.byref(cache.c),
                                                _ptr(kv_proj), token_count, base_pos,
                                                _ptr(positions), int(bool(is_k))))


def encode_turboquant_attention(stream: Stream, tq: TurboQuantModel, cache: TurboQuantKvCache, q,
                                num_heads: int, seq_len: int, out, attn_scale: float | None = None,
                                seq_lens=None, num_splits: int = 0):
    """turboquant_attention + fused_sdpa_reduce (attention.rs:394-489)."""
    if attn_scale is None:
        attn_scale = 1.0 / math.sqrt(cache.head_dim)  # mil-rs/src/weights.rs:210-217
    check(lib.imh_encode_turboquant_attention(stream.handle, tq.handle, C.byref(cache.c), _ptr(q),
                                              num_heads, seq_len, _ptr(seq_lens), attn_scale,
                                              _ptr(out), num_splits))


def encode_kv_cache_and_attention(stream: Stream, tq: TurboQuantModel, cache: TurboQuantKvCache,
                                  k_proj, v_proj, q, num_heads: int, seq_pos: int, out,
                                  attn_scale: float | None = None):
    """encode_kv_cache_and_attention (attention.rs:117-610), decode step."""
    if attn_scale is None:
        attn_scale = 1.0 / math.sqrt(cache.head_dim)
    check(lib.imh_encode_kv_cache_and_attention(stream.handle, tq.handle, C.byref(cache.c),
                                                _ptr(k_proj), _ptr(v_proj), _ptr(q), num_heads,
                                                seq_pos, attn_scale, _ptr(out)))


class Fp16KvCache:
    """One layer of the FP16 KV cache (attention.rs:492-496) for `batch` sequences:
    k, v [batch, num_kv_heads, max_seq_len, head_dim] f16."""

    def __init__(self, dev: Device, batch: int, num_kv_heads: int, head_dim: int, max_seq_len: int):
        self.batch, self.num_kv_heads, self.head_dim, self.max_seq_len = (
            batch, num_kv_heads, head_dim, max_seq_len)
        shp = (batch, num_kv_heads, max_seq_len, head_dim)
        self.k = dev.empty(shp, np.float16)
        self.v = dev.empty(shp, np.float16)
        self._c = _lib.Fp16KvCache(self.k.ptr, self.v.ptr, batch, num_kv_heads, head_dim, max_seq_len)

    @property
    def c(self):
        return self._c

    def zero(self, stream: Stream):
        stream.zero(self.k)
        stream.zero(self.v)


def encode_kv_scatter(stream: Stream, cache: Fp16KvCache, proj, token_count: int, base_pos: int,
                      is_k: bool, positions=None):
    """encode_kv_scatter (ops/kv.rs:35-58) into the K or V array."""
    check(lib.imh_encode_kv_scatter(stream.handle, C.byref(cache.c), _ptr(proj), token_count, base_pos,
                                    _ptr(positions), int(bool(is_k))))


def encode_fp16_attention(stream: Stream, cache: Fp16KvCache, q, num_heads: int, seq_len: int, out,
                          token_count: int = 1, attn_scale: float | None = None, seq_lens=None,
                          num_splits: int = 0):
    """fused_sdpa / FlashDecoding split + reduce (attention_ops.rs:274-417)."""
    if attn_scale is None:
        attn_scale = 1.0 / math.sqrt(cache.head_dim)
    check(lib.imh_encode_fp16_attention(stream.handle, C.byref(cache.c), _ptr(q), num_heads, token_count,
                                        seq_len, _ptr(seq_lens), attn_scale, _ptr(out), num_splits))


def encode_fp16_kv_cache_and_attention(stream: Stream, cache: Fp16KvCache, k_proj, v_proj, q,
                                       num_heads: int, seq_pos: int, out, token_count: int = 1,
                                       attn_scale: float | None = None):
    """The FP16 branch of encode_kv_cache_and_attention (attention.rs:491-607)."""
    if attn_scale is None:
        attn_scale = 1.0 / math.sqrt(cache.head_dim)
    check(lib.imh_encode_fp16_kv_cache_and_attention(stream.handle, C.byref(cache.c), _ptr(k_proj),
                                                     _ptr(v_proj), _ptr(q), num_heads, token_count,
                                                     seq_pos, attn_scale, _ptr(out)))


__all__ = [
    "AffineQuantizedWeight", "encode_projection", "encode_batched_affine_matvec_int4",
    "encode_fused_ffn_gate_up_act_int4", "encode_fused_residual_norm_affine_matvec_int4",
    "TurboQuantModel", "TurboQuantKvCache", "encode_turboquant_cache_write",
    "encode_turboquant_attention", "encode_kv_cache_and_attention", "Fp16KvCache", "encode_kv_scatter",
    "encode_fp16_attention", "encode_fp16_kv_cache_and_attention", "_lib",
]
