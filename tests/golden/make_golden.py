"""Writes the golden fixtures in this directory from the CPU oracle.

The reference (Rust) cannot be built or run here, so these vectors come from
the oracle's restatement of the reference's CPU path, pinned by the checks in
tests/test_oracle.py.  They freeze that restatement: tests/test_golden.py
re-derives every fixture with the oracle (bit for bit) and runs the GPU path
against them.

    python tests/golden/make_golden.py      # rewrites *.npz here

Fixtures (all seeded):
  int4_cfg1.npz  W [1024,1024] f16 ~ N(0, 0.02), group 128:
                 packed codes, f32 and f16 scales/zeros, x [1,1024], y [1,1024]
  int4_awq.npz   W [64,256] with AWQ scales ~ U[0.5, 2], x [4,256], y [4,64]
  tq.npz         TurboQuant tables (d=128, 8 bits, seed 42), the K and V cache
                 write of 4 tokens x 2 kv heads, and a ctx-300 attention case
                 (8 query heads, GQA 4:1)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402


def int4_cfg1():
    rng = np.random.default_rng(20260101)
    n = k = 1024
    w16 = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    packed, sc, zp = O.quantize_tensor_int4(w16.astype(np.float32), 128)
    x16 = rng.standard_normal((1, k)).astype(np.float16)
    wdq = O.dequant_affine_int4(packed, sc, zp, n, k, 128)
    y = O.matvec_f16w(wdq, x16)
    return dict(w16=w16, packed=packed, scales=sc, zeros=zp, scales16=O.convert_params_to_f16(sc),
                zeros16=O.convert_params_to_f16(zp), x16=x16, y=y)


def int4_awq():
    rng = np.random.default_rng(20260102)
    n, k, b = 64, 256, 4
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16).astype(np.float32)
    s = rng.uniform(0.5, 2.0, k).astype(np.float32)
    packed, sc, zp = O.quantize_tensor_int4((w * s[None, :]).astype(np.float32), 128)
    awq16 = s.astype(np.float16)
    x16 = rng.standard_normal((b, k)).astype(np.float16)
    wdq = O.dequant_affine_int4(packed, sc, zp, n, k, 128)
    y = O.matvec_f16w(wdq, x16, awq16)
    return dict(w=w, awq=s, awq16=awq16, packed=packed, scales=sc, zeros=zp, x16=x16, y=y)


def tq():
    t = O.TQTables(128, 8, 42)
    rng = np.random.default_rng(20260103)
    kv_k = rng.standard_normal((1, 4, 2, 128)).astype(np.float16)
    kv_v = rng.standard_normal((1, 4, 2, 128)).astype(np.float16)
    kc, ks, kr = O.tq_cache_write(kv_k, t, True, 8)
    vc, vs, _ = O.tq_cache_write(kv_v, t, False, 8)
    # attention: 300 positions of K/V for 2 kv heads, 8 query heads
    ctx, max_seq = 300, 320
    ak = rng.standard_normal((1, ctx, 2, 128)).astype(np.float16)
    av = rng.standard_normal((1, ctx, 2, 128)).astype(np.float16)
    akc, aks, akr = O.tq_cache_write(ak, t, True, max_seq)
    avc, avs, _ = O.tq_cache_write(av, t, False, max_seq)
    q = rng.standard_normal((1, 8, 128)).astype(np.float16)
    scale = np.float32(1.0 / np.sqrt(128.0))
    out = O.tq_attention(q, t, akc, avc, aks, avs, akr, ctx, float(scale))
    return dict(signs=t.signs, k_codebook=t.k_codebook, k_bounds=t.k_bounds, v_codebook=t.v_codebook,
                v_bounds=t.v_bounds, qjl=t.qjl, write_k_in=kv_k, write_v_in=kv_v, write_k_codes=kc,
                write_k_scales=ks, write_k_rnorms=kr, write_v_codes=vc, write_v_scales=vs,
                attn_k_in=ak, attn_v_in=av, attn_q=q, attn_scale=scale, attn_ctx=np.int32(ctx),
                attn_max_seq=np.int32(max_seq), attn_out=out)


BUILDERS = {"int4_cfg1": int4_cfg1, "int4_awq": int4_awq, "tq": tq}

if __name__ == "__main__":
    for name, fn in BUILDERS.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(path, os.path.getsize(path))
