"""Host-side INT4 weight quantizer producing the layout the kernels consume.

Vectorised restatement of ironmill-compile's JIT INT4 path:
``quantize_tensor_int4`` (ironmill-compile/src/weights/quantized.rs:408-465) over
``quantize_affine`` (mil-rs/src/ir/passes/affine_quantize.rs:256-298), nibble
packing low-first (int4_pack.rs:20-34), AWQ column scaling
(quantized.rs:912-1010, ``W * s`` quantized, ``s`` stored as f16) and the GPU
upload conversion of scales/zeros to f16 (core/dequant.rs:305-345,
metal/weights.rs:1064-1092).  Every f32 operation matches the Rust order, so
codes, scales and zeros are bit-identical to the reference path.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GROUP_SIZE = 128


def _round_half_away(x: np.ndarray) -> np.ndarray:
    """Rust f32::round (ties away from zero), exactly, in f32."""
    t = np.trunc(x)
    frac = np.abs(x - t)  # exact for f32
    # np.where keeps the sign of a truncated -0.0 (Rust: (-0.25f32).round() == -0.0)
    return np.where(frac >= np.float32(0.5), t + np.sign(x), t).astype(np.float32)


def quantize_groups(g: np.ndarray, qmax: float = 15.0):
    """quantize_affine over rows of ``g`` [n_groups, group_len] (all finite).

    Returns (codes u8 [n_groups, group_len], scale f32 [n_groups], zp f32 [n_groups]).
    """
    g = np.asarray(g, np.float32)
    finite = np.isfinite(g)
    mn = np.where(finite, g, np.float32(np.inf)).min(axis=1).astype(np.float32)
    mx = np.where(finite, g, np.float32(-np.inf)).max(axis=1).astype(np.float32)
    none = ~np.isfinite(mn) | ~np.isfinite(mx)
    rng = (mx - mn).astype(np.float32)
    degenerate = np.abs(rng) < np.finfo(np.float32).eps
    with np.errstate(divide="ignore", invalid="ignore"):
        s_regular = (rng / np.float32(qmax)).astype(np.float32)
        scale = np.where(degenerate, np.float32(1.0), s_regular).astype(np.float32)
        zp = np.where(degenerate, _round_half_away(-mn), _round_half_away((-mn / scale).astype(np.float32)))
        zp = zp.astype(np.float32)
        t = _round_half_away(((g / scale[:, None]).astype(np.float32) + zp[:, None]).astype(np.float32))
    t = np.where(np.isnan(t), np.float32(0), t)
    q = np.clip(t, 0, qmax).astype(np.uint8)
    q[none] = 0
    scale = np.where(none, np.float32(1.0), scale).astype(np.float32)
    zp = np.where(none, np.float32(0.0), zp).astype(np.float32)
    return q, scale, zp


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """Two codes per byte, element 2i in the low nibble (int4_pack.rs:20-34)."""
    c = np.asarray(codes, np.uint8).reshape(-1)
    if c.size % 2:
        c = np.concatenate([c, np.zeros(1, np.uint8)])
    return ((c[1::2] & 0x0F) << 4 | (c[0::2] & 0x0F)).astype(np.uint8)


@dataclass
class QuantizedInt4:
    """Host copy of one INT4 weight in the GPU upload layout."""

    data: np.ndarray       # u8 [n, k/2]
    scales: np.ndarray     # f16 [n, k/gs]
    zeros: np.ndarray      # f16 [n, k/gs]
    scales_f32: np.ndarray  # f32 [n, k/gs] as produced by the quantizer (the CPU dequant path)
    zeros_f32: np.ndarray
    awq: np.ndarray | None  # f16 [k] or None
    n: int
    k: int
    group_size: int = GROUP_SIZE


@dataclass
class QuantizedInt8:
    """Host copy of one INT8 weight in the GPU upload layout (one code byte per element)."""

    data: np.ndarray       # u8 [n, k]
    scales: np.ndarray     # f16 [n, k/gs]
    zeros: np.ndarray      # f16 [n, k/gs]
    scales_f32: np.ndarray
    zeros_f32: np.ndarray
    awq: np.ndarray | None
    n: int
    k: int
    group_size: int = GROUP_SIZE


def quantize_int8(w: np.ndarray, group_size: int = GROUP_SIZE, awq_scales=None) -> QuantizedInt8:
    """quantize_tensor_int8 (quantized.rs:852-901): the INT4 rule with qmax 255, no packing."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    if k % group_size:
        raise ValueError(f"k={k} must be a multiple of group_size={group_size}")
    awq16 = None
    if awq_scales is not None:
        s = np.asarray(awq_scales, np.float32)
        w = (w * s[None, :]).astype(np.float32)
        awq16 = s.astype(np.float16)
    q, sc, zp = quantize_groups(w.reshape(n * (k // group_size), group_size), qmax=255.0)
    sc = sc.reshape(n, k // group_size)
    zp = zp.reshape(n, k // group_size)
    return QuantizedInt8(data=q.reshape(n, k), scales=sc.astype(np.float16), zeros=zp.astype(np.float16),
                         scales_f32=sc, zeros_f32=zp, awq=awq16, n=n, k=k, group_size=group_size)


def quantize_int4(w: np.ndarray, group_size: int = GROUP_SIZE, awq_scales=None) -> QuantizedInt4:
    """quantize_tensor_int4 (+ AWQ): w f32/f16 [n, k], k a multiple of group_size."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    if k % group_size:
        raise ValueError(f"k={k} must be a multiple of group_size={group_size}")
    awq16 = None
    if awq_scales is not None:
        s = np.asarray(awq_scales, np.float32)
        w = (w * s[None, :]).astype(np.float32)  # quantized.rs:936-950
        awq16 = s.astype(np.float16)               # quantized.rs:994-1007
    g = w.reshape(n * (k // group_size), group_size)
    q, sc, zp = quantize_groups(g)
    data = pack_int4(q).reshape(n, k // 2)
    sc = sc.reshape(n, k // group_size)
    zp = zp.reshape(n, k // group_size)
    return QuantizedInt4(data=data, scales=sc.astype(np.float16), zeros=zp.astype(np.float16),
                         scales_f32=sc, zeros_f32=zp, awq=awq16, n=n, k=k, group_size=group_size)
