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
from ._lib import AffineInt8Weight as _AffineInt8Weight
from ._lib import (AffineInt4Weight, DecoderConfig, DecoderLayerWeights, FusedResidualNormParams, QkNormRopeParams,
                   TqKvCache, check, lib)
from .quant import QuantizedInt4, QuantizedInt8
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


class AffineInt8Weight:
    """Device copy of an INT8 weight (quantize_tensor_int8, quantized.rs:852-901)."""

    def __init__(self, dev: Device, q: QuantizedInt8):
        self.n, self.k, self.group_size = q.n, q.k, q.group_size
        self.data = dev.upload(q.data)
        self.scales = dev.upload(q.scales)
        self.zeros = dev.upload(q.zeros)
        self.awq_scales = dev.upload(q.awq) if q.awq is not None else None
        self._c = _AffineInt8Weight(self.data.ptr, self.scales.ptr, self.zeros.ptr,
                                    self.awq_scales.ptr if self.awq_scales is not None else None,
                                    self.n, self.k, self.group_size)

    @property
    def c(self) -> _AffineInt8Weight:
        return self._c


def encode_projection_int8(stream: Stream, x, weight: AffineInt8Weight, y, token_count: int):
    """superblock_matvec_int8 (affine_matvec.metal:123-189) over token_count rows, f16 in and out."""
    check(lib.imh_encode_affine_projection_int8(stream.handle, _ptr(x), token_count, C.byref(weight.c), _ptr(y)))


def encode_quantize_input_q8(stream: Stream, x, token_count: int, k: int, q8, q8_scales):
    """quantize_input_q8 (quantize.metal:21-52) per 128-element group of each row."""
    check(lib.imh_encode_quantize_input_q8(stream.handle, _ptr(x), token_count, k, _ptr(q8), _ptr(q8_scales)))


def encode_affine_matvec_int4xq8(stream: Stream, q8, q8_scales, token_count: int, weight: AffineQuantizedWeight, y):
    """superblock_affine_matvec_int4xq8 (affine_fused.metal:115-176) on Q8 activations."""
    check(lib.imh_encode_affine_matvec_int4xq8(stream.handle, _ptr(q8), _ptr(q8_scales), token_count,
                                               C.byref(weight.c), _ptr(y)))


def encode_projection_int4_q8(stream: Stream, x, weight: AffineQuantizedWeight, y, token_count: int,
                              q8_out=None, q8_scales_out=None):
    """The decode projection on Q8 activations quantized from the f16 rows x in the same launch
    (quantize.metal:21-52 then affine_fused.metal:115-176; pipeline.rs:639-664); optionally
    writes the codes / scales for the layer's other projections."""
    check(lib.imh_encode_affine_projection_int4_q8(stream.handle, _ptr(x), token_count, C.byref(weight.c), _ptr(y),
                                                   _ptr(q8_out), _ptr(q8_scales_out)))


PROBE_TILE, PROBE_FLAT, PROBE_BAND = 0, 1, 2


def diag_stream_read(stream: Stream, src, n: int, k: int, sink, mode=PROBE_TILE, nmat=1, rows=16, tiles=1,
                     waves=4, grid=0, threads=0):
    """Streaming probe (no reference counterpart): reads the INT4 weight bytes at src with no
    compute.  TILE: `tiles` tiles of `rows` rows of each of `nmat` n x k weights per workgroup,
    `waves` waves per weight (rows 16 is the INT4 matvec's own pattern).  FLAT: `grid`
    workgroups of `threads` threads reading contiguous runs of the n x k weight.  BAND: the
    row-band matvec's launch, `grid` workgroups each reading one band of rows of each weight."""
    shape = _lib.ProbeShape(mode, nmat, rows, tiles, waves, grid, threads)
    check(lib.imh_diag_stream_read(stream.handle, _ptr(src), n, k, C.byref(shape), _ptr(sink)))


def diag_valu_matvec(stream: Stream, x, weight: AffineQuantizedWeight, y, token_count: int):
    """VALU-dot INT4 matvec (no reference counterpart): the projection's semantics computed
    as a wavefront-reduction matvec with in-register dequant, for the counter A/B against the
    MFMA kernels.  k in {2560, 4096}, token_count <= 8."""
    check(lib.imh_diag_valu_matvec(stream.handle, _ptr(x), token_count, C.byref(weight.c), _ptr(y)))


def kv_positions(seq_pos: int, token_count: int, window_size: int, max_seq_len: int) -> dict:
    """The cache positions of one step (imh_kv_positions_for; attention.rs:141-163): the
    layer cache's stride (its max_seq_len), the write position, the attention base and the
    seq_len to give the attention ops."""
    out = _lib.KvPositions()
    check(lib.imh_kv_positions_for(seq_pos, token_count, window_size, max_seq_len, C.byref(out)))
    return {"stride": out.stride, "write_pos": out.write_pos, "attn_base": out.attn_base, "attn_len": out.attn_len}


GEMM_F16, GEMM_BF16, GEMM_FP8_E4M3 = 0, 1, 2


def encode_affine_gemm_int4(stream: Stream, x, token_count: int, weight: AffineQuantizedWeight, y,
                            precision: int = GEMM_BF16):
    """superblock_matmul_int4 (affine_matmul.metal:10-152) at a chosen matrix-core precision:
    GEMM_F16 (x, y f16: the projection op), GEMM_BF16 (x, y bf16) or GEMM_FP8_E4M3 (x, y bf16,
    x / awq rounded to e4m3).  bf16 data travels as uint16 bit patterns."""
    check(lib.imh_affine_gemm_int4(stream.handle, _ptr(x), token_count, C.byref(weight.c), _ptr(y), precision))


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


def encode_ffn_block_int4(stream: Stream, x, gate: AffineQuantizedWeight, up: AffineQuantizedWeight,
                          down: AffineQuantizedWeight, act_out, y, token_count: int = 1, use_gelu: bool = False):
    """encode_ffn_block (metal/ffn.rs:13-144): act_out = act(x.Wg) * (x.Wu), y = act_out . Wd^T."""
    check(lib.imh_encode_ffn_block_int4(stream.handle, _ptr(x), token_count, C.byref(gate.c), C.byref(up.c),
                                        C.byref(down.c), _ptr(act_out), _ptr(y), int(bool(use_gelu))))


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


def encode_turboquant_cache_write_kv(stream: Stream, tq: TurboQuantModel, cache: TurboQuantKvCache,
                                    k_proj, v_proj, token_count: int, base_pos: int, positions=None):
    """Both cache writes of attention.rs:344-391 in one launch."""
    check(lib.imh_encode_turboquant_cache_write_kv(stream.handle, tq.handle, C.byref(cache.c), _ptr(k_proj),
                                                   _ptr(v_proj), token_count, base_pos, _ptr(positions)))


def encode_turboquant_attention(stream: Stream, tq: TurboQuantModel, cache: TurboQuantKvCache, q,
                                num_heads: int, seq_len: int, out, attn_scale: float | None = None,
                                seq_lens=None, num_splits: int = 0, token_count: int = 1):
    """turboquant_attention + fused_sdpa_reduce (attention.rs:394-489).  token_count > 1:
    q / out [batch][token_count][heads][d], token t attends causally to positions
    < seq_len - token_count + t + 1 (turboquant.metal:268, token_idx = tgid.y)."""
    if attn_scale is None:
        attn_scale = 1.0 / math.sqrt(cache.head_dim)  # mil-rs/src/weights.rs:210-217
    if token_count != 1:
        check(lib.imh_encode_turboquant_attention_tokens(stream.handle, tq.handle, C.byref(cache.c), _ptr(q),
                                                         num_heads, token_count, seq_len, _ptr(seq_lens),
                                                         attn_scale, _ptr(out), num_splits))
        return
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


# ------------------------------------------------------------ decode-step glue


def read_device(dev: Device, ptr: int, shape, dtype) -> np.ndarray:
    """Copy device memory handed out by pointer (e.g. a decoder's KV cache) to the host."""
    out = np.empty(shape, dtype)
    check(lib.imh_copy_to_host(dev.handle, out.ctypes.data_as(C.c_void_p), ptr, out.nbytes))
    return out


def encode_rms_norm(stream: Stream, x, weight, out, hidden_size: int, token_count: int, eps: float):
    """rms_norm (normalization.metal:19-57)."""
    check(lib.imh_encode_rms_norm(stream.handle, _ptr(x), _ptr(weight), _ptr(out), hidden_size, token_count, eps))


def encode_fused_residual_rms_norm(stream: Stream, a, b, weight, normed_output, residual_output,
                                   hidden_size: int, token_count: int, eps: float):
    """fused_residual_rms_norm (fused_residual_norm.metal:33-75)."""
    check(lib.imh_encode_fused_residual_rms_norm(stream.handle, _ptr(a), _ptr(b), _ptr(weight), _ptr(normed_output),
                                                 _ptr(residual_output), hidden_size, token_count, eps))


def encode_residual_add(stream: Stream, a, b, out, n: int):
    check(lib.imh_encode_residual_add(stream.handle, _ptr(a), _ptr(b), _ptr(out), n))


def encode_fused_embedding_norm(stream: Stream, token_ids, embedding, norm_weight, normed_output, raw_output,
                                hidden_size: int, token_count: int, vocab_size: int, eps: float,
                                embed_scale: float = 1.0):
    """fused_embedding_norm (fused_embedding_norm.metal:29-73)."""
    check(lib.imh_encode_fused_embedding_norm(stream.handle, _ptr(token_ids), _ptr(embedding), _ptr(norm_weight),
                                              _ptr(normed_output), _ptr(raw_output), hidden_size, token_count,
                                              vocab_size, eps, embed_scale))


def rope_cache(head_dim: int, max_pos: int, theta: float, rotary_dim: int = 0):
    """precompute_rope_cache (ironmill-core/src/rope.rs:22-50) -> (cos, sin) f16 [max_pos, head_dim/2]."""
    cos = np.empty((max_pos, head_dim // 2), np.float16)
    sin = np.empty_like(cos)
    check(lib.imh_rope_cache_fill(head_dim, max_pos, theta, rotary_dim, cos.ctypes.data_as(C.c_void_p),
                                  sin.ctypes.data_as(C.c_void_p)))
    return cos, sin


def encode_qk_norm_rope(stream: Stream, q, k, cos_cache, sin_cache, num_heads: int, num_kv_heads: int,
                        head_dim: int, max_pos: int, q_norm=None, k_norm=None, rotary_dim: int = 0,
                        seq_offset: int = 0, positions=None, batch: int = 1, token_count: int = 1,
                        eps: float = 1e-6):
    """encode_qk_norm_and_rope (metal/attention.rs:26-92), in place on q and k."""
    p = QkNormRopeParams(_ptr(q), _ptr(k), _ptr(q_norm), _ptr(k_norm), _ptr(cos_cache), _ptr(sin_cache), num_heads,
                         num_kv_heads, head_dim, rotary_dim, max_pos, seq_offset, _ptr(positions), batch,
                         token_count, eps)
    check(lib.imh_encode_qk_norm_rope(stream.handle, C.byref(p)))


class Decoder:
    """One decode step of a pre-norm transformer over INT4 weights and a TurboQuant
    or FP16 KV cache (MetalInference::decode_step, metal/engine.rs:178-180 ->
    run_pipeline_inner, metal/pipeline.rs:228-1313), for `batch` sequences."""

    def __init__(self, dev: Device, *, hidden_size, intermediate_size, num_layers, num_heads, num_kv_heads,
                 head_dim, vocab_size, max_seq_len, batch=1, rotary_dim=0, rms_eps=1e-6, rope_theta=1e6,
                 attn_scale=0.0, embed_scale=0.0, use_gelu=False, kv_cache="turboquant", tq_seed=42,
                 window_sizes=None):
        self.dev = dev
        kind = {"turboquant": _lib.IMH_KV_TURBOQUANT, "fp16": _lib.IMH_KV_FP16}[kv_cache]
        self.kv_kind = kv_cache
        # per-layer sliding windows (0 = full attention), copied by the library at creation
        win = None if window_sizes is None else np.ascontiguousarray(window_sizes, np.uint32)
        if win is not None and win.size != num_layers:
            raise ValueError("window_sizes needs one entry per layer")
        self.cfg = DecoderConfig(hidden_size, intermediate_size, num_layers, num_heads, num_kv_heads, head_dim,
                                 vocab_size, max_seq_len, batch, rotary_dim, rms_eps, attn_scale, embed_scale,
                                 int(bool(use_gelu)), kind, rope_theta, tq_seed,
                                 None if win is None else win.ctypes.data)
        h = C.c_void_p()
        check(lib.imh_decoder_create(dev.handle, C.byref(self.cfg), C.byref(h)))
        self._h = h
        self._keep = {}

    @property
    def handle(self):
        return self._h

    def set_layer(self, layer: int, *, input_norm, post_attn_norm, q_proj, k_proj, v_proj, o_proj, gate_proj,
                  up_proj, down_proj, q_norm=None, k_norm=None):
        w = DecoderLayerWeights(_ptr(input_norm), _ptr(post_attn_norm), _ptr(q_norm), _ptr(k_norm), q_proj.c,
                                k_proj.c, v_proj.c, o_proj.c, gate_proj.c, up_proj.c, down_proj.c)
        check(lib.imh_decoder_set_layer(self._h, layer, C.byref(w)))
        self._keep[layer] = (input_norm, post_attn_norm, q_norm, k_norm, q_proj, k_proj, v_proj, o_proj,
                             gate_proj, up_proj, down_proj)

    def set_model(self, embedding, final_norm, lm_head: AffineQuantizedWeight):
        check(lib.imh_decoder_set_model(self._h, _ptr(embedding), _ptr(final_norm), C.byref(lm_head.c)))
        self._keep["model"] = (embedding, final_norm, lm_head)

    def reset(self, stream: Stream, positions=None):
        if positions is not None:
            pos = np.ascontiguousarray(positions, np.int32)
            check(lib.imh_decoder_reset(self._h, stream.handle, pos.ctypes.data_as(C.c_void_p)))
        else:
            check(lib.imh_decoder_reset(self._h, stream.handle, None))

    def step(self, stream: Stream, token_ids, logits):
        check(lib.imh_decoder_step(self._h, stream.handle, _ptr(token_ids), _ptr(logits)))

    def prefill(self, stream: Stream, token_ids, token_count: int, logits):
        """token_count tokens per sequence (token_ids [batch, token_count]) at the current
        positions; logits of each sequence's last token (run_pipeline_inner, token_count > 1)."""
        check(lib.imh_decoder_prefill(self._h, stream.handle, _ptr(token_ids), token_count, _ptr(logits)))

    def write_kv(self, stream: Stream, layer: int, k_proj, v_proj, token_count: int, base_pos: int = 0):
        """Write K/V projections [batch, token_count, nkv, head_dim] of one layer into its cache."""
        check(lib.imh_decoder_write_kv(self._h, stream.handle, layer, _ptr(k_proj), _ptr(v_proj), token_count,
                                       base_pos))

    def positions(self) -> np.ndarray:
        """Host mirror of the positions (advanced by eager steps only)."""
        out = np.empty(self.cfg.batch, np.int32)
        check(lib.imh_decoder_positions(self._h, out.ctypes.data_as(C.c_void_p)))
        return out

    def sync_positions(self, stream: Stream) -> np.ndarray:
        """Device positions after every encoded step and graph replay; raises
        IronmillError (IMH_ERANGE) if a step ran past the cache's end."""
        out = np.empty(self.cfg.batch, np.int32)
        check(lib.imh_decoder_sync_positions(self._h, stream.handle, out.ctypes.data_as(C.c_void_p)))
        return out

    def set_tq_tables(self, tables: "TurboQuantModel"):
        """Use caller-built TurboQuant tables (TurboQuantModel(dev, host_tables=...))."""
        check(lib.imh_decoder_set_tq_tables(self._h, tables.handle))
        self._keep["tq_tables"] = tables

    def kv_cache(self, layer: int) -> dict:
        """Host copies of one layer's cache arrays ([batch, kv heads, slots, ...]; a windowed
        layer has window_size slots)."""
        c = self.cfg
        if self.kv_kind == "turboquant":
            t = TqKvCache()
            check(lib.imh_decoder_kv_cache(self._h, layer, C.byref(t), None))
            shp = (c.batch, c.num_kv_heads, t.max_seq_len)
            return {"k_codes": read_device(self.dev, t.k_codes, shp + (c.head_dim,), np.uint8),
                    "v_codes": read_device(self.dev, t.v_codes, shp + (c.head_dim,), np.uint8),
                    "k_scales": read_device(self.dev, t.k_scales, shp, np.float32),
                    "v_scales": read_device(self.dev, t.v_scales, shp, np.float32),
                    "k_r_norms": read_device(self.dev, t.k_r_norms, shp, np.float32)}
        f = _lib.Fp16KvCache()
        check(lib.imh_decoder_kv_cache(self._h, layer, None, C.byref(f)))
        shp = (c.batch, c.num_kv_heads, f.max_seq_len)
        return {"k": read_device(self.dev, f.k, shp + (c.head_dim,), np.float16),
                "v": read_device(self.dev, f.v, shp + (c.head_dim,), np.float16)}

    def close(self):
        if getattr(self, "_h", None):
            lib.imh_decoder_free(self._h)
            self._h = None

    def __del__(self):
        self.close()


__all__ = [
    "AffineQuantizedWeight", "encode_projection", "encode_affine_gemm_int4", "GEMM_F16", "GEMM_BF16",
    "GEMM_FP8_E4M3", "encode_batched_affine_matvec_int4",
    "encode_fused_ffn_gate_up_act_int4", "encode_fused_residual_norm_affine_matvec_int4",
    "TurboQuantModel", "TurboQuantKvCache", "encode_turboquant_cache_write", "encode_turboquant_cache_write_kv",
    "encode_turboquant_attention", "encode_kv_cache_and_attention", "Fp16KvCache", "encode_kv_scatter",
    "encode_fp16_attention", "encode_fp16_kv_cache_and_attention", "read_device", "encode_rms_norm",
    "encode_fused_residual_rms_norm", "encode_residual_add", "encode_fused_embedding_norm", "rope_cache",
    "encode_qk_norm_rope", "Decoder", "_lib",
]
