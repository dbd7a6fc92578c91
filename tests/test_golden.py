"""The committed golden fixtures (tests/golden/make_golden.py).

CPU: the oracle and the library's host quantizer re-derive every fixture bit
for bit, so a change to either shows up here before it reaches a GPU run.
GPU: the library's ops reproduce the fixtures -- INT4 projections within the
BASELINE tolerance, TurboQuant codes bit for bit (caller-provided tables),
attention within tolerance with and without a KV split.
"""
import os

import numpy as np
import pytest

import oracle as O
from conftest import assert_close
from ironmill_amd import ops, quant

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint8)


# ---------------------------------------------------------------- CPU


def test_cfg1_oracle_reproduces_fixture():
    g = load("int4_cfg1")
    packed, sc, zp = O.quantize_tensor_int4(g["w16"].astype(np.float32), 128)
    assert np.array_equal(packed, g["packed"])
    assert np.array_equal(bits(sc), bits(g["scales"])) and np.array_equal(bits(zp), bits(g["zeros"]))
    assert np.array_equal(bits(O.convert_params_to_f16(sc)), bits(g["scales16"]))
    wdq = O.dequant_affine_int4(packed, sc, zp, 1024, 1024, 128)
    assert np.array_equal(bits(O.matvec_f16w(wdq, g["x16"])), bits(g["y"]))


def test_cfg1_host_quantizer_matches_fixture():
    g = load("int4_cfg1")
    q = quant.quantize_int4(g["w16"])
    assert np.array_equal(q.data, g["packed"].reshape(q.data.shape))
    assert np.array_equal(bits(q.scales), bits(g["scales16"].reshape(q.scales.shape)))
    assert np.array_equal(bits(q.zeros), bits(g["zeros16"].reshape(q.zeros.shape)))


def test_awq_oracle_reproduces_fixture():
    g = load("int4_awq")
    packed, sc, zp = O.quantize_tensor_int4((g["w"] * g["awq"][None, :]).astype(np.float32), 128)
    assert np.array_equal(packed, g["packed"])
    wdq = O.dequant_affine_int4(packed, sc, zp, 64, 256, 128)
    assert np.array_equal(bits(O.matvec_f16w(wdq, g["x16"], g["awq16"])), bits(g["y"]))
    q = quant.quantize_int4(g["w"], awq_scales=g["awq"])
    assert np.array_equal(q.data, g["packed"].reshape(q.data.shape))


def test_tq_oracle_reproduces_fixture():
    g = load("tq")
    t = O.TQTables(128, 8, 42)
    for name in ("signs", "k_codebook", "k_bounds", "v_codebook", "v_bounds", "qjl"):
        assert np.array_equal(bits(getattr(t, name)), bits(g[name])), name
    kc, ks, kr = O.tq_cache_write(g["write_k_in"], t, True, 8)
    vc, vs, _ = O.tq_cache_write(g["write_v_in"], t, False, 8)
    assert np.array_equal(kc, g["write_k_codes"]) and np.array_equal(vc, g["write_v_codes"])
    assert np.array_equal(bits(ks), bits(g["write_k_scales"])) and np.array_equal(bits(kr), bits(g["write_k_rnorms"]))
    assert np.array_equal(bits(vs), bits(g["write_v_scales"]))
    ms = int(g["attn_max_seq"])
    akc, aks, akr = O.tq_cache_write(g["attn_k_in"], t, True, ms)
    avc, avs, _ = O.tq_cache_write(g["attn_v_in"], t, False, ms)
    out = O.tq_attention(g["attn_q"], t, akc, avc, aks, avs, akr, int(g["attn_ctx"]), float(g["attn_scale"]))
    assert np.array_equal(bits(out), bits(g["attn_out"]))


# ---------------------------------------------------------------- GPU


def upload_fixture_weight(dev, packed, scales, zeros, n, k, awq=None):
    q = quant.QuantizedInt4(data=packed.reshape(n, k // 2), scales=scales.reshape(n, k // 128),
                            zeros=zeros.reshape(n, k // 128), scales_f32=None, zeros_f32=None,
                            awq=awq, n=n, k=k)
    return ops.AffineQuantizedWeight(dev, q)


@pytest.mark.gpu
def test_gpu_cfg1_projection(dev, stream):
    g = load("int4_cfg1")
    w = upload_fixture_weight(dev, g["packed"], g["scales16"], g["zeros16"], 1024, 1024)
    xd, yd = dev.upload(g["x16"]), dev.empty((1, 1024), np.float16)
    ops.encode_projection(stream, xd, w, yd, 1)
    stream.sync()
    assert_close(yd.read(), g["y"], what="cfg1 golden", ulps=2)


@pytest.mark.gpu
def test_gpu_awq_projection(dev, stream):
    g = load("int4_awq")
    w = upload_fixture_weight(dev, g["packed"], O.convert_params_to_f16(g["scales"]),
                              O.convert_params_to_f16(g["zeros"]), 64, 256, awq=g["awq16"])
    xd, yd = dev.upload(g["x16"]), dev.empty((4, 64), np.float16)
    ops.encode_projection(stream, xd, w, yd, 4)
    stream.sync()
    assert_close(yd.read(), g["y"], what="awq golden", ulps=2)


@pytest.mark.gpu
def test_gpu_tq_write_and_attention(dev, stream):
    g = load("tq")
    tq = ops.TurboQuantModel(dev, 128, 8, 42, host_tables={k: g[k] for k in (
        "signs", "k_codebook", "k_bounds", "v_codebook", "v_bounds", "qjl")})
    cache = ops.TurboQuantKvCache(dev, 1, 2, 128, 8)
    cache.zero(stream)
    ops.encode_turboquant_cache_write(stream, tq, cache, dev.upload(g["write_k_in"]), 4, 0, True)
    ops.encode_turboquant_cache_write(stream, tq, cache, dev.upload(g["write_v_in"]), 4, 0, False)
    stream.sync()
    assert np.array_equal(cache.k_codes.read(), g["write_k_codes"])
    assert np.array_equal(cache.v_codes.read(), g["write_v_codes"])
    assert np.array_equal(bits(cache.k_scales.read()), bits(g["write_k_scales"]))
    assert np.array_equal(bits(cache.k_r_norms.read()), bits(g["write_k_rnorms"]))
    assert np.array_equal(bits(cache.v_scales.read()), bits(g["write_v_scales"]))

    ctx, ms = int(g["attn_ctx"]), int(g["attn_max_seq"])
    ac = ops.TurboQuantKvCache(dev, 1, 2, 128, ms)
    ac.zero(stream)
    ops.encode_turboquant_cache_write(stream, tq, ac, dev.upload(g["attn_k_in"]), ctx, 0, True)
    ops.encode_turboquant_cache_write(stream, tq, ac, dev.upload(g["attn_v_in"]), ctx, 0, False)
    qd = dev.upload(g["attn_q"])
    for splits in (1, 4):
        out = dev.empty((1, 8, 128), np.float16)
        ops.encode_turboquant_attention(stream, tq, ac, qd, 8, ctx, out, float(g["attn_scale"]),
                                        num_splits=splits)
        stream.sync()
        assert_close(out.read(), g["attn_out"], what=f"tq golden splits={splits}")
