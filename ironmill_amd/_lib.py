"""ctypes binding of libironmill_hip.so (the C ABI in include/ironmill_hip.h).

The shared library is the product: every op runs there.  There is no Python
or CPU fallback -- if the library is missing, importing this module raises.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# IRONMILL_HIP_LIB selects another build of the same library (e.g. a debug build)
LIB_PATH = os.environ.get("IRONMILL_HIP_LIB") or os.path.join(_HERE, "lib", "libironmill_hip.so")

IMH_OK = 0
IMH_EINVAL = -1
IMH_EUNSUPPORTED = -2
IMH_EDEVICE = -3
IMH_ENOMEM = -4
IMH_ERANGE = -5

ERROR_NAMES = {
    IMH_EINVAL: "IMH_EINVAL",
    IMH_EUNSUPPORTED: "IMH_EUNSUPPORTED",
    IMH_EDEVICE: "IMH_EDEVICE",
    IMH_ENOMEM: "IMH_ENOMEM",
    IMH_ERANGE: "IMH_ERANGE",
}

IMH_TQ_SIGNS, IMH_TQ_K_CODEBOOK, IMH_TQ_K_BOUNDS, IMH_TQ_V_CODEBOOK, IMH_TQ_V_BOUNDS, IMH_TQ_QJL = range(6)


class IronmillError(RuntimeError):
    """A non-zero status from the C ABI, with the library's own message."""

    def __init__(self, code: int, message: str):
        self.code = code
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")


class DeviceInfo(C.Structure):
    _fields_ = [
        ("ordinal", C.c_int),
        ("compute_units", C.c_int),
        ("wavefront_size", C.c_int),
        ("clock_khz", C.c_int),
        ("total_global_mem", C.c_size_t),
        ("lds_per_block", C.c_size_t),
        ("arch", C.c_char * 64),
    ]


class AffineInt4Weight(C.Structure):
    """imh_affine_int4_weight (AffineQuantizedWeight, metal/weights.rs:129-147)."""

    _fields_ = [
        ("data", C.c_void_p),
        ("scales", C.c_void_p),
        ("zeros", C.c_void_p),
        ("awq_scales", C.c_void_p),
        ("n", C.c_uint32),
        ("k", C.c_uint32),
        ("group_size", C.c_uint32),
    ]


class AffineInt8Weight(C.Structure):
    """imh_affine_int8_weight (the INT8 weight, quantized.rs:852-901)."""

    _fields_ = AffineInt4Weight._fields_


class ProbeShape(C.Structure):
    """imh_probe_shape (the streaming probe's launch shape; no reference counterpart)."""

    _fields_ = [(f, C.c_uint32) for f in ("mode", "nmat", "rows", "tiles", "waves", "grid", "threads")]


class FusedResidualNormParams(C.Structure):
    """imh_fused_residual_norm_params (FusedResidualNormAffineInt4Params, ops/fused.rs:45-66)."""

    _fields_ = [
        ("a", C.c_void_p),
        ("b", C.c_void_p),
        ("norm_weight", C.c_void_p),
        ("residual_output", C.c_void_p),
        ("weight", C.POINTER(AffineInt4Weight)),
        ("output", C.c_void_p),
        ("normed_output", C.c_void_p),
        ("token_count", C.c_uint32),
        ("eps", C.c_float),
    ]


class TqKvCache(C.Structure):
    """imh_tq_kv_cache (one layer of MetalKvCache, metal/turboquant/cache.rs:45-96)."""

    _fields_ = [
        ("k_codes", C.c_void_p),
        ("v_codes", C.c_void_p),
        ("k_scales", C.c_void_p),
        ("v_scales", C.c_void_p),
        ("k_r_norms", C.c_void_p),
        ("batch", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("max_seq_len", C.c_uint32),
    ]


class Fp16KvCache(C.Structure):
    """imh_fp16_kv_cache (one layer of the FP16 KV cache, attention.rs:492-496)."""

    _fields_ = [
        ("k", C.c_void_p),
        ("v", C.c_void_p),
        ("batch", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("max_seq_len", C.c_uint32),
    ]


class QkNormRopeParams(C.Structure):
    """imh_qk_norm_rope_params (QkNormAndRopeParams, metal/attention.rs:12-24)."""

    _fields_ = [
        ("q", C.c_void_p),
        ("k", C.c_void_p),
        ("q_norm", C.c_void_p),
        ("k_norm", C.c_void_p),
        ("cos_cache", C.c_void_p),
        ("sin_cache", C.c_void_p),
        ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("rotary_dim", C.c_uint32),
        ("max_pos", C.c_uint32),
        ("seq_offset", C.c_uint32),
        ("positions", C.c_void_p),
        ("batch", C.c_uint32),
        ("token_count", C.c_uint32),
        ("eps", C.c_float),
    ]


class DecoderConfig(C.Structure):
    """imh_decoder_config."""

    _fields_ = [
        ("hidden_size", C.c_uint32),
        ("intermediate_size", C.c_uint32),
        ("num_layers", C.c_uint32),
        ("num_heads", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("vocab_size", C.c_uint32),
        ("max_seq_len", C.c_uint32),
        ("batch", C.c_uint32),
        ("rotary_dim", C.c_uint32),
        ("rms_eps", C.c_float),
        ("attn_scale", C.c_float),
        ("embed_scale", C.c_float),
        ("use_gelu", C.c_int),
        ("kv_cache", C.c_int),
        ("rope_theta", C.c_double),
        ("tq_seed", C.c_uint64),
        ("window_sizes", C.c_void_p),
    ]


class KvPositions(C.Structure):
    """imh_kv_positions (KvCacheAndAttentionParams positions, attention.rs:141-163)."""

    _fields_ = [(f, C.c_uint32) for f in ("stride", "write_pos", "attn_base", "attn_len")]


class DecoderLayerWeights(C.Structure):
    """imh_decoder_layer_weights."""

    _fields_ = [
        ("input_norm", C.c_void_p),
        ("post_attn_norm", C.c_void_p),
        ("q_norm", C.c_void_p),
        ("k_norm", C.c_void_p),
        ("q_proj", AffineInt4Weight),
        ("k_proj", AffineInt4Weight),
        ("v_proj", AffineInt4Weight),
        ("o_proj", AffineInt4Weight),
        ("gate_proj", AffineInt4Weight),
        ("up_proj", AffineInt4Weight),
        ("down_proj", AffineInt4Weight),
    ]


IMH_KV_TURBOQUANT = 0
IMH_KV_FP16 = 1

P = C.c_void_p
U32 = C.c_uint32
SZ = C.c_size_t
I = C.c_int

# name -> (restype, argtypes); kept in the order of include/ironmill_hip.h
SIGNATURES = {
    "imh_last_error": (C.c_char_p, []),
    "imh_device_count": (I, [C.POINTER(I)]),
    "imh_device_open": (I, [I, C.POINTER(P)]),
    "imh_device_free": (None, [P]),
    "imh_device_get_info": (I, [P, C.POINTER(DeviceInfo)]),
    "imh_buffer_alloc": (I, [P, SZ, C.POINTER(P)]),
    "imh_buffer_alloc_with_data": (I, [P, P, SZ, C.POINTER(P)]),
    "imh_buffer_free": (None, [P]),
    "imh_buffer_length": (SZ, [P]),
    "imh_buffer_device_ptr": (P, [P]),
    "imh_buffer_write": (I, [P, SZ, P, SZ]),
    "imh_buffer_read": (I, [P, SZ, P, SZ]),
    "imh_copy_to_host": (I, [P, P, P, SZ]),
    "imh_stream_create": (I, [P, C.POINTER(P)]),
    "imh_stream_free": (None, [P]),
    "imh_stream_sync": (I, [P]),
    "imh_stream_native": (P, [P]),
    "imh_fill_zero": (I, [P, P, SZ]),
    "imh_stream_begin_capture": (I, [P]),
    "imh_stream_end_capture": (I, [P, C.POINTER(P)]),
    "imh_graph_launch": (I, [P, P]),
    "imh_graph_free": (None, [P]),
    "imh_event_create": (I, [P, C.POINTER(P)]),
    "imh_event_free": (None, [P]),
    "imh_event_record": (I, [P, P]),
    "imh_event_elapsed_ms": (I, [P, P, C.POINTER(C.c_float)]),
    "imh_encode_affine_projection_int4": (I, [P, P, U32, C.POINTER(AffineInt4Weight), P]),
    "imh_encode_batched_affine_matvec_int4": (I, [P, P, U32, C.POINTER(AffineInt4Weight), P,
                                                  C.POINTER(AffineInt4Weight), P]),
    "imh_encode_fused_ffn_gate_up_act_int4": (I, [P, P, U32, C.POINTER(AffineInt4Weight),
                                                  C.POINTER(AffineInt4Weight), P, I]),
    "imh_encode_ffn_block_int4": (I, [P, P, U32, C.POINTER(AffineInt4Weight), C.POINTER(AffineInt4Weight),
                                      C.POINTER(AffineInt4Weight), P, P, I]),
    "imh_affine_gemm_int4": (I, [P, P, U32, C.POINTER(AffineInt4Weight), P, I]),
    "imh_encode_affine_projection_int8": (I, [P, P, U32, C.POINTER(AffineInt8Weight), P]),
    "imh_kv_positions_for": (I, [U32, U32, U32, U32, C.POINTER(KvPositions)]),
    "imh_diag_stream_read": (I, [P, P, U32, U32, C.POINTER(ProbeShape), P]),
    "imh_diag_valu_matvec": (I, [P, P, U32, C.POINTER(AffineInt4Weight), P]),
    "imh_encode_quantize_input_q8": (I, [P, P, U32, U32, P, P]),
    "imh_encode_affine_matvec_int4xq8": (I, [P, P, P, U32, C.POINTER(AffineInt4Weight), P]),
    "imh_encode_affine_projection_int4_q8": (I, [P, P, U32, C.POINTER(AffineInt4Weight), P, P, P]),
    "imh_encode_fused_residual_norm_affine_matvec_int4": (I, [P, C.POINTER(FusedResidualNormParams)]),
    "imh_tq_tables_create": (I, [P, U32, U32, C.c_uint64, C.POINTER(P)]),
    "imh_tq_tables_create_from_host": (I, [P, U32, U32, P, P, P, P, P, P, C.POINTER(P)]),
    "imh_tq_tables_free": (None, [P]),
    "imh_tq_tables_read": (I, [P, I, P, SZ, C.POINTER(SZ)]),
    "imh_tq_cache_sizes": (I, [U32, U32, U32, U32, C.POINTER(SZ), C.POINTER(SZ)]),
    "imh_encode_turboquant_cache_write": (I, [P, P, C.POINTER(TqKvCache), P, U32, U32, P, I]),
    "imh_encode_turboquant_cache_write_kv": (I, [P, P, C.POINTER(TqKvCache), P, P, U32, U32, P]),
    "imh_encode_turboquant_attention": (I, [P, P, C.POINTER(TqKvCache), P, U32, U32, P, C.c_float, P,
                                            U32]),
    "imh_encode_turboquant_attention_noalloc": (I, [P, P, C.POINTER(TqKvCache), P, U32, U32, P, C.c_float, P,
                                                    U32]),
    "imh_encode_turboquant_attention_tokens": (I, [P, P, C.POINTER(TqKvCache), P, U32, U32, U32, P, C.c_float, P,
                                            U32]),
    "imh_encode_kv_cache_and_attention": (I, [P, P, C.POINTER(TqKvCache), P, P, P, U32, U32, C.c_float,
                                              P]),
    "imh_encode_rms_norm": (I, [P, P, P, P, U32, U32, C.c_float]),
    "imh_encode_fused_residual_rms_norm": (I, [P, P, P, P, P, P, U32, U32, C.c_float]),
    "imh_encode_residual_add": (I, [P, P, P, P, SZ]),
    "imh_encode_fused_embedding_norm": (I, [P, P, P, P, P, P, U32, U32, U32, C.c_float, C.c_float]),
    "imh_rope_cache_fill": (I, [U32, U32, C.c_double, U32, P, P]),
    "imh_encode_qk_norm_rope": (I, [P, C.POINTER(QkNormRopeParams)]),
    "imh_encode_kv_scatter": (I, [P, C.POINTER(Fp16KvCache), P, U32, U32, P, I]),
    "imh_encode_fp16_attention": (I, [P, C.POINTER(Fp16KvCache), P, U32, U32, U32, P, C.c_float, P, U32]),
    "imh_encode_fp16_kv_cache_and_attention": (I, [P, C.POINTER(Fp16KvCache), P, P, P, U32, U32, U32,
                                                   C.c_float, P]),
    "imh_decoder_create": (I, [P, C.POINTER(DecoderConfig), C.POINTER(P)]),
    "imh_decoder_free": (None, [P]),
    "imh_decoder_set_layer": (I, [P, U32, C.POINTER(DecoderLayerWeights)]),
    "imh_decoder_set_model": (I, [P, P, P, C.POINTER(AffineInt4Weight)]),
    "imh_decoder_reset": (I, [P, P, P]),
    "imh_decoder_step": (I, [P, P, P, P]),
    "imh_decoder_prefill": (I, [P, P, P, U32, P]),
    "imh_decoder_write_kv": (I, [P, P, U32, P, P, U32, U32]),
    "imh_decoder_positions": (I, [P, P]),
    "imh_decoder_sync_positions": (I, [P, P, P]),
    "imh_decoder_set_tq_tables": (I, [P, P]),
    "imh_decoder_kv_cache": (I, [P, U32, C.POINTER(TqKvCache), C.POINTER(Fp16KvCache)]),
    "imh_decoder_tq_tables": (I, [P, C.POINTER(P)]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libironmill_hip.so not found at {LIB_PATH}; build it with "
            "`python ironmill_amd/build.py` (hipcc, gfx950)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def last_error() -> str:
    msg = lib.imh_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(rc: int) -> None:
    if rc != IMH_OK:
        raise IronmillError(rc, last_error())
