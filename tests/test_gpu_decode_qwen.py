"""The decode step at the Qwen3-4B attention layout, free-running against the oracle.

Config: hidden 2560, 32 query / 8 KV heads of 128, four layers (intermediate
2048 and vocabulary 2048 keep the CPU oracle fast), a cache prefilled with 200
positions of K/V rows (configs[2] distribution), then three decode steps in
which both sides write their own cache rows from their own K/V projections.

What the logits can be held to.  Every activation is stored as f16 between
ops, so two correct implementations that sum in different orders round some
stored values one f16 step apart, and four layers of the random model amplify
those steps.  The oracle measures this on itself (the CPU-only study in
tests/test_decode_sensitivity.py): the same math with float32 instead of
float64 sums already moves the logits by ~1e-3 with either cache (more with
TurboQuant at short contexts, where a one-step change of a K/V value can move
it across a codebook boundary or flip a QJL sign).  So the GPU is compared with
  B  -- the oracle with the GPU upload's weight semantics ((q - z16) * s16,
        exact) summing in float64, and
  A  -- the reference's CPU path (dequantized weights rounded to f16, f32 sums),
and the bound is the oracle's own spread, measured in the same test
(conftest.assert_decoder_logits):
  rel(GPU, B) <= max(1e-3, 2 rel(B32, B), rel(A, B)),
  rel(GPU, A) <= that + rel(A, B),
where B32 is B summing in float32.  A systematic error (a wrong index, scale
or sign) moves the logits by far more than that spread.  The spreads are held
to conftest.SPREAD_CAP (2e-3), so the bound cannot loosen with the data: on
these inputs (prefill 200, batch 1, 2 and 8, either cache) rel(B32, B)
measures 0.90-1.38e-3 and rel(A, B) 1.31-1.76e-3 per step on the CPU.
"""
import numpy as np
import pytest

import oracle as O
from conftest import assert_decoder_logits
from decoder_models import host_model, kv_rows
from ironmill_amd import ops

pytestmark = pytest.mark.gpu

CFG = dict(hidden_size=2560, intermediate_size=2048, num_layers=4, num_heads=32, num_kv_heads=8, head_dim=128,
           vocab_size=2048, max_seq_len=512, rms_eps=1e-6, rope_theta=1e6)
PREFILL = 200
STEPS = 3


@pytest.fixture(scope="module")
def model():
    return host_model(4242, CFG)


def device_model(dev, model):
    layers, emb, fnorm, lm = model
    dev_layers = []
    for hl in layers:
        dl = {k: dev.upload(hl[k]) for k in ("input_norm", "post_attn_norm", "q_norm", "k_norm")}
        q = ops.AffineQuantizedWeight(dev, hl["q_proj"])

        def shared(name, owner):
            w = hl[name]
            return ops.AffineQuantizedWeight.from_pointers(dev.upload(w.data), dev.upload(w.scales),
                                                           dev.upload(w.zeros), owner.awq_scales, w.n, w.k)

        dl.update(q_proj=q, k_proj=shared("k_proj", q), v_proj=shared("v_proj", q),
                  o_proj=ops.AffineQuantizedWeight(dev, hl["o_proj"]))
        g = ops.AffineQuantizedWeight(dev, hl["gate_proj"])
        dl.update(gate_proj=g, up_proj=shared("up_proj", g), down_proj=ops.AffineQuantizedWeight(dev, hl["down_proj"]))
        dev_layers.append(dl)
    return dev_layers, dev.upload(emb), dev.upload(fnorm), ops.AffineQuantizedWeight(dev, lm)


@pytest.mark.parametrize("kv_cache,batch", [("fp16", 1), ("turboquant", 1), ("fp16", 2), ("turboquant", 2),
                                            ("fp16", 8), ("turboquant", 8)])
def test_decoder_qwen_layout_free_running(dev, stream, model, kv_cache, batch):
    cfg = dict(CFG, batch=batch)
    print(f"decoder qwen layout kv={kv_cache} batch={batch}", flush=True)
    layers, emb, fnorm, lm = model
    dl, demb, dfn, dlm = device_model(dev, model)
    d = ops.Decoder(dev, kv_cache=kv_cache, **cfg)
    for l, w in enumerate(dl):
        d.set_layer(l, **w)
    d.set_model(demb, dfn, dlm)

    refs = {"A": O.DecoderReference(cfg, layers, emb, fnorm, lm, kv_cache=kv_cache),
            "B": O.DecoderReference(cfg, layers, emb, fnorm, lm, kv_cache=kv_cache, weights="exact", acc="f64"),
            "B32": O.DecoderReference(cfg, layers, emb, fnorm, lm, kv_cache=kv_cache, weights="exact", acc="f32")}

    # the same prefilled context on every side: GPU rows written by imh_decoder_write_kv,
    # oracle rows by its own cache write (bit-exact with the GPU's on equal inputs)
    rng = np.random.default_rng(99 + batch)
    for l in range(cfg["num_layers"]):
        k, v = kv_rows(rng, batch, PREFILL, 8), kv_rows(rng, batch, PREFILL, 8)
        d.write_kv(stream, l, dev.upload(k), dev.upload(v), PREFILL, 0)
        if kv_cache == "turboquant":
            tabs = refs["A"].tables
            kc, ks, kr = O.tq_cache_write(k, tabs, True, cfg["max_seq_len"])
            vc, vs, _ = O.tq_cache_write(v, tabs, False, cfg["max_seq_len"])
            rows = dict(k_codes=kc, v_codes=vc, k_scales=ks, v_scales=vs, k_r_norms=kr)
        else:
            rows = dict(k=np.zeros_like(refs["A"].caches[l]["k"]), v=np.zeros_like(refs["A"].caches[l]["v"]))
            rows["k"][:, :, :PREFILL] = k.transpose(0, 2, 1, 3)
            rows["v"][:, :, :PREFILL] = v.transpose(0, 2, 1, 3)
        for r in refs.values():
            for name, arr in rows.items():
                r.caches[l][name][...] = arr
    # sequences continue at different positions (the later ones overwrite prefilled rows)
    start = (PREFILL - 23 * np.arange(batch)).astype(np.int32)
    d.reset(stream, start)
    for r in refs.values():
        r.positions = start.copy()

    logits = dev.empty((batch, cfg["vocab_size"]), np.float16)
    for step in range(STEPS):
        tok = rng.integers(0, cfg["vocab_size"], batch).astype(np.uint32)
        d.step(stream, dev.upload(tok), logits)
        stream.sync()
        want = {name: r.step(tok.astype(np.int64)) for name, r in refs.items()}
        assert_decoder_logits(logits.read(), want["A"], want["B"], want["B32"], f"  step {step}")
    assert np.array_equal(d.sync_positions(stream), start + STEPS)
