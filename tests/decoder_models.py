"""Seeded random decoder models for the decode-step tests (host side only).

Weights are W ~ N(0, std) quantized INT4 group 128 with AWQ scales ~U[0.5, 2]
(BASELINE.json configs[1] and [4] distributions).  Large models are quantized
with the oracle's C quantizer, which is bit-identical to the host quantizer
(tests/test_host.py, tests/test_golden.py) and ~30x faster; the result is the
same QuantizedInt4 record the upload takes.
"""
import numpy as np

import oracle as O
from ironmill_amd import quant


def q4(w: np.ndarray, awq=None) -> quant.QuantizedInt4:
    """quantize_tensor_int4 (+ AWQ) of w [n, k] through the oracle's C quantizer."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    awq16 = None
    if awq is not None:
        s = np.asarray(awq, np.float32)
        w = (w * s[None, :]).astype(np.float32)
        awq16 = s.astype(np.float16)
    packed, sc, zp = O.quantize_tensor_int4(w, 128)
    return quant.QuantizedInt4(data=packed.reshape(n, k // 2), scales=sc.astype(np.float16),
                               zeros=zp.astype(np.float16), scales_f32=sc, zeros_f32=zp, awq=awq16, n=n, k=k)


def host_model(seed: int, cfg: dict, std: float = 0.02, qk_norm: bool = True):
    """(layers, embedding f16, final norm f16, lm_head) with Q/K/V and gate/up sharing
    one AWQ vector per layer (as AWQ exports do: they scale one activation)."""
    rng = np.random.default_rng(seed)
    H, F, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    qd, kvd = cfg["num_heads"] * cfg["head_dim"], cfg["num_kv_heads"] * cfg["head_dim"]

    def w(n, k):
        return (rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)).astype(np.float32)

    def norm(n):
        return rng.uniform(0.8, 1.2, n).astype(np.float16)

    layers = []
    for _ in range(cfg["num_layers"]):
        s_in = rng.uniform(0.5, 2.0, H).astype(np.float32)
        s_f = rng.uniform(0.5, 2.0, F).astype(np.float32)
        layers.append(dict(input_norm=norm(H), post_attn_norm=norm(H),
                           q_norm=norm(cfg["head_dim"]) if qk_norm else None,
                           k_norm=norm(cfg["head_dim"]) if qk_norm else None,
                           q_proj=q4(w(qd, H), s_in), k_proj=q4(w(kvd, H), s_in), v_proj=q4(w(kvd, H), s_in),
                           o_proj=q4(w(H, qd)), gate_proj=q4(w(F, H), s_in), up_proj=q4(w(F, H), s_in),
                           down_proj=q4(w(H, F), s_f)))
    emb = rng.standard_normal((V, H), dtype=np.float32).astype(np.float16)
    return layers, emb, norm(H), q4(w(V, H))


def kv_rows(rng, batch, tokens, nkv, hd=128):
    """K/V rows f16 N(0,1) with 4 outlier channels per head x10."""
    x = rng.standard_normal((batch, tokens, nkv, hd), dtype=np.float32)
    for h in range(nkv):
        x[:, :, h, rng.choice(hd, 4, replace=False)] *= 10.0
    return x.astype(np.float16)


QWEN3_4B = dict(hidden_size=2560, intermediate_size=9728, num_layers=36, num_heads=32, num_kv_heads=8, head_dim=128,
                vocab_size=151936, rms_eps=1e-6, rope_theta=1e6)


def shared_layer_model(seed: int, cfg: dict, std: float = 0.02):
    """A model of cfg's full shape whose layers all hold one layer's weights (quantized from
    N(0, std), AWQ as in host_model): every layer still runs every launch on its own cache and
    activations, while the oracle dequantizes one layer instead of num_layers."""
    one = dict(cfg, num_layers=1)
    layers, emb, fnorm, lm = host_model(seed, one, std)
    return [layers[0]] * cfg["num_layers"], emb, fnorm, lm


def block_kv(rng, batch, block, nkv, hd=128):
    """K and V rows [batch, block, nkv, hd] of one cache block (configs[2] distribution)."""
    return kv_rows(rng, batch, block, nkv, hd), kv_rows(rng, batch, block, nkv, hd)
