"""The `.ironml-gpu` bundle reader (ironmill_amd.bundle) on bundles in the reference's layout.

CPU: a bundle written by write_bundle (the layout of write_gpu_bundle,
ironmill-compile/src/gpu/bundle.rs:51-296) reads back bit for bit; a manifest
shaped exactly like the reference's own test bundle
(metal/bundle.rs:351-427: no scale/zero dtypes, which default to float16)
parses; the f16 upload conversion equals the oracle's convert_params_to_f16;
malformed bundles raise.  GPU: a projection from bundle-loaded weights
matches the oracle, and a decoder loaded from a bundle computes the same
logits, bit for bit, as one built from the same arrays directly.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
from ironmill_amd import bundle as B
from ironmill_amd import quant

CONFIG = {"architecture": "qwen3", "hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2,
          "num_attention_heads": 4, "num_key_value_heads": 1, "head_dim": 128, "vocab_size": 512,
          "max_position_embeddings": 64, "rms_norm_eps": 1e-6, "rope_theta": 1e6, "tie_word_embeddings": False}


def model_tensors(seed=3, cfg=CONFIG):
    rng = np.random.default_rng(seed)
    H, F, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    qd, kvd = cfg["num_attention_heads"] * cfg["head_dim"], cfg["num_key_value_heads"] * cfg["head_dim"]

    def q4(n, k, awq=None):
        return quant.quantize_int4((rng.standard_normal((n, k)) * 0.05).astype(np.float32), awq_scales=awq)

    def norm(n):
        return rng.uniform(0.8, 1.2, n).astype(np.float16)

    t = {"model.embed_tokens.weight": rng.standard_normal((V, H)).astype(np.float16),
         "model.norm.weight": norm(H), "lm_head.weight": q4(V, H)}
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}"
        s_in = rng.uniform(0.5, 2.0, H).astype(np.float32)
        t.update({f"{p}.input_layernorm.weight": norm(H), f"{p}.post_attention_layernorm.weight": norm(H),
                  f"{p}.self_attn.q_norm.weight": norm(cfg["head_dim"]),
                  f"{p}.self_attn.k_norm.weight": norm(cfg["head_dim"]),
                  f"{p}.self_attn.q_proj.weight": q4(qd, H, s_in), f"{p}.self_attn.k_proj.weight": q4(kvd, H, s_in),
                  f"{p}.self_attn.v_proj.weight": q4(kvd, H, s_in), f"{p}.self_attn.o_proj.weight": q4(H, qd),
                  f"{p}.mlp.gate_proj.weight": q4(F, H, s_in), f"{p}.mlp.up_proj.weight": q4(F, H, s_in),
                  f"{p}.mlp.down_proj.weight": q4(H, F, rng.uniform(0.5, 2.0, F).astype(np.float32))})
    return t


def test_round_trip(tmp_path):
    path = str(tmp_path / "m.ironml-gpu")
    tensors = model_tensors()
    B.write_bundle(path, CONFIG, tensors)
    b = B.GpuBundle(path)
    assert b.config == CONFIG
    assert sorted(b.tensor_names()) == sorted(tensors)
    m = json.load(open(os.path.join(path, "manifest.json")))
    assert m["format_version"] == 1 and m["quantization"]["method"] == "affine"
    e = m["tensors"]["model.layers.0.self_attn.q_proj.weight"]
    assert e["format"] == "affine_dequantize" and e["quantized_data_file"] == "weights/model_layers_0_self_attn_q_proj_weight.qdata"
    assert e["scale_dtype"] == "float32" and e["axis"] == 1 and e["group_size"] == 128 and "awq_scales_file" in e
    for name, t in tensors.items():
        if isinstance(t, quant.QuantizedInt4):
            q = b.affine_int4(name)
            assert np.array_equal(q.data, t.data)
            assert np.array_equal(q.scales_f32.view(np.uint32), t.scales_f32.view(np.uint32))
            assert np.array_equal(q.zeros_f32.view(np.uint32), t.zeros_f32.view(np.uint32))
            # the upload conversion: convert_params_to_f16 (f32 -> f16, round to nearest even)
            assert np.array_equal(q.scales.view(np.uint16), O.convert_params_to_f16(t.scales_f32).view(np.uint16).reshape(q.scales.shape))
            assert np.array_equal(q.zeros.view(np.uint16), O.convert_params_to_f16(t.zeros_f32).view(np.uint16).reshape(q.zeros.shape))
            assert (q.awq is None) == (t.awq is None)
            if t.awq is not None:
                assert np.array_equal(q.awq.view(np.uint16), t.awq.view(np.uint16))
        else:
            assert np.array_equal(b.dense_f16(name).view(np.uint16), t.view(np.uint16))


def test_reference_shaped_manifest(tmp_path):
    """The manifest of the reference's own reader test (metal/bundle.rs:351-427): f16 scale
    and zero files without dtype fields, which default to float16."""
    path = tmp_path / "test.ironml-gpu"
    (path / "weights").mkdir(parents=True)
    n, k = 16, 256
    codes = np.random.default_rng(1).integers(0, 256, n * k // 2).astype(np.uint8)
    sc = np.full(n * 2, 0.01, np.float16)
    zp = np.full(n * 2, 7.0, np.float16)
    (path / "weights" / "g.qdata").write_bytes(codes.tobytes())
    (path / "weights" / "g.scale").write_bytes(sc.tobytes())
    (path / "weights" / "g.zeros").write_bytes(zp.tobytes())
    manifest = {"format_version": 1,
                "model_config": {**CONFIG, "architecture": "llama", "extra": {}},
                "quantization": {"method": "none", "n_bits": 16, "seed": 42, "min_elements": 1024},
                "tensors": {"model.layers.0.mlp.gate_proj.weight": {
                    "format": "affine_dequantize", "quantized_data_file": "weights/g.qdata",
                    "scales_file": "weights/g.scale", "zeros_file": "weights/g.zeros", "shape": [n, k],
                    "bit_width": 4, "group_size": 128, "axis": 1, "dtype": "uint8"}}}
    (path / "manifest.json").write_text(json.dumps(manifest, indent=2))
    q = B.GpuBundle(str(path)).affine_int4("model.layers.0.mlp.gate_proj.weight")
    assert np.array_equal(q.data.reshape(-1), codes)
    assert np.array_equal(q.scales.reshape(-1).view(np.uint16), sc.view(np.uint16))
    assert np.array_equal(q.zeros.reshape(-1).view(np.uint16), zp.view(np.uint16))


def test_errors(tmp_path):
    with pytest.raises(B.BundleError, match="failed to read manifest"):
        B.GpuBundle(str(tmp_path / "missing.ironml-gpu"))
    path = str(tmp_path / "v2.ironml-gpu")
    B.write_bundle(path, CONFIG, {"model.norm.weight": np.ones(4, np.float16)})
    m = json.load(open(os.path.join(path, "manifest.json")))
    m["format_version"] = 2
    json.dump(m, open(os.path.join(path, "manifest.json"), "w"))
    with pytest.raises(B.BundleError, match="format version"):
        B.GpuBundle(path)
    m["format_version"] = 1
    del m["model_config"]["hidden_size"]
    json.dump(m, open(os.path.join(path, "manifest.json"), "w"))
    with pytest.raises(B.BundleError, match="hidden_size"):
        B.GpuBundle(path)
    ok = str(tmp_path / "ok.ironml-gpu")
    B.write_bundle(ok, CONFIG, {"model.norm.weight": np.ones(4, np.float16)})
    b = B.GpuBundle(ok)
    with pytest.raises(B.BundleError, match="not found"):
        b.tensor("lm_head.weight")
    with pytest.raises(B.BundleError, match="not INT4 affine"):
        b.affine_int4("model.norm.weight")


@pytest.mark.gpu
def test_bundle_projection_matches_oracle(tmp_path, dev, stream):
    from conftest import assert_close
    from ironmill_amd import ops
    path = str(tmp_path / "p.ironml-gpu")
    rng = np.random.default_rng(9)
    s = rng.uniform(0.5, 2.0, 1024).astype(np.float32)
    w = (rng.standard_normal((768, 1024)) * 0.02).astype(np.float32)
    B.write_bundle(path, CONFIG, {"w": quant.quantize_int4(w, awq_scales=s)})
    q = B.GpuBundle(path).affine_int4("w")
    wt = ops.AffineQuantizedWeight(dev, q)
    x = rng.standard_normal((3, 1024)).astype(np.float16)
    y = dev.empty((3, 768), np.float16)
    ops.encode_projection(stream, dev.upload(x), wt, y, 3)
    stream.sync()
    packed, sc, zp = O.quantize_tensor_int4((w * s[None, :]).astype(np.float32), 128)
    ref = O.matvec_f16w(O.dequant_affine_int4(packed, sc, zp, 768, 1024), x, s.astype(np.float16))
    assert_close(y.read(), ref, what="bundle projection", ulps=2)


@pytest.mark.gpu
def test_bundle_decoder_matches_direct(tmp_path, dev, stream):
    """load_decoder over a bundle gives the logits of a decoder built from the same arrays,
    bit for bit (same kernels, same launches: the AWQ vectors are shared by content)."""
    from ironmill_amd import ops
    path = str(tmp_path / "d.ironml-gpu")
    tensors = model_tensors(5)
    B.write_bundle(path, CONFIG, tensors)
    a = B.load_decoder(dev, B.GpuBundle(path), max_seq_len=64, batch=2)
    b = ops.Decoder(dev, hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4, num_kv_heads=1,
                    head_dim=128, vocab_size=512, max_seq_len=64, batch=2, rms_eps=1e-6, rope_theta=1e6)
    keep = []

    def w(name):
        x = ops.AffineQuantizedWeight(dev, B.GpuBundle(path).affine_int4(name))
        keep.append(x)
        return x

    shared = {}
    for i in range(2):
        p = f"model.layers.{i}"
        qw = w(f"{p}.self_attn.q_proj.weight")
        gw = w(f"{p}.mlp.gate_proj.weight")

        def sh(name, owner):
            t = B.GpuBundle(path).affine_int4(name)
            x = ops.AffineQuantizedWeight.from_pointers(dev.upload(t.data), dev.upload(t.scales), dev.upload(t.zeros),
                                                        owner.awq_scales, t.n, t.k)
            keep.append(x)
            return x

        d = {k: dev.upload(tensors[f"{p}.{k2}.weight"]) for k, k2 in (
            ("input_norm", "input_layernorm"), ("post_attn_norm", "post_attention_layernorm"),
            ("q_norm", "self_attn.q_norm"), ("k_norm", "self_attn.k_norm"))}
        keep.append(d)
        b.set_layer(i, q_proj=qw, k_proj=sh(f"{p}.self_attn.k_proj.weight", qw), v_proj=sh(f"{p}.self_attn.v_proj.weight", qw),
                    o_proj=w(f"{p}.self_attn.o_proj.weight"), gate_proj=gw, up_proj=sh(f"{p}.mlp.up_proj.weight", gw),
                    down_proj=w(f"{p}.mlp.down_proj.weight"), **d)
    emb, fn = dev.upload(tensors["model.embed_tokens.weight"]), dev.upload(tensors["model.norm.weight"])
    b.set_model(emb, fn, w("lm_head.weight"))
    la, lb = dev.empty((2, 512), np.float16), dev.empty((2, 512), np.float16)
    tok = dev.upload(np.array([3, 77], np.uint32))
    for dec in (a, b):
        dec.reset(stream, np.array([0, 5], np.int32))
    for step in range(3):
        a.step(stream, tok, la)
        b.step(stream, tok, lb)
        stream.sync()
        assert np.array_equal(la.read().view(np.uint16), lb.read().view(np.uint16)), f"step {step}"
