"""GPU parity of sliding-window attention layers in the decode step.

The decoder keeps a windowed layer's cache as a ring of W slots (the buffer
stride, write position and attention bound of attention.rs:141-163 and
turboquant/cache.rs:382-400); the oracle (DecoderReference with window_sizes)
keeps a linear cache and attends to the last W positions of each sequence, the
definition the ring implements.  Layers 1 and 2 use windows of 5 and 3
positions, layer 0 full attention; two sequences start at positions 0 and 9
and decode 10 tokens, so both rings wrap several times.  At every step the
logits must stay within the north star's rel-L2 1e-3 of the oracle on the GPU
upload's weight semantics (weights="exact": (q - z16) * s16, f64 sums) --
or the oracle's own spreads where they are larger: twice its f32-vs-f64
distance, or the reference CPU path's distance from it
(conftest.assert_decoder_logits; ten free-running steps reach ~1.05e-3) --
and within that bound plus the CPU path's distance from the exact oracle
against the CPU path (f16-dequantized weights): this model's logits move by
~1e-3 between those two weight semantics alone (measured 0.8-1.2e-3 per
step, with and without windows), so 1e-3 against the CPU path is not a bound
the semantics allow here.  With the TurboQuant cache
the oracle takes the code rows the GPU wrote (slot p % W of a windowed layer
holds position p), as in the full-attention decoder test: the cache write is
bit-exact on equal inputs, and rounding differences in its input can move a
vector across a codebook boundary.
"""
import numpy as np
import pytest

import oracle as O
from conftest import assert_decoder_logits, rel_l2
from ironmill_amd import IronmillError, ops
from test_gpu_decode import CFG, make_model

pytestmark = pytest.mark.gpu

WINDOWS = [0, 5, 3]


def build(dev, model, kv_cache, windows, cfg=CFG):
    host_layers, dev_layers, emb, fnorm, lm = model
    d = ops.Decoder(dev, kv_cache=kv_cache, window_sizes=windows, **cfg)
    for l, dl in enumerate(dev_layers):
        d.set_layer(l, **{k: v for k, v in dl.items() if not k.startswith("_")})
    d._keep_lm = ops.AffineQuantizedWeight(dev, lm)
    d.set_model(dev.upload(emb), dev.upload(fnorm), d._keep_lm)
    return d


@pytest.mark.parametrize("kv_cache,batch", [("fp16", 2), ("turboquant", 2), ("fp16", 1), ("turboquant", 1)])
def test_decoder_sliding_window_matches_reference(dev, stream, kv_cache, batch):
    cfg = dict(CFG, batch=batch)
    model = make_model(dev, 91)
    d = build(dev, model, kv_cache, WINDOWS, cfg)
    host_layers, _, emb, fnorm, lm = model
    ref = O.DecoderReference(cfg, host_layers, emb, fnorm, lm, kv_cache=kv_cache, window_sizes=WINDOWS)
    exact = O.DecoderReference(cfg, host_layers, emb, fnorm, lm, kv_cache=kv_cache, window_sizes=WINDOWS,
                               weights="exact", acc="f64")
    exact32 = O.DecoderReference(cfg, host_layers, emb, fnorm, lm, kv_cache=kv_cache, window_sizes=WINDOWS,
                                 weights="exact", acc="f32")
    start = np.array([0, 9] if batch == 2 else [9], np.int32)
    d.reset(stream, start)
    for r in (ref, exact, exact32):
        r.positions = start.copy()
    rng = np.random.default_rng(6 if batch == 2 else 7)
    logits = dev.empty((batch, cfg["vocab_size"]), np.float16)

    def force_rows(l, cache, pos):
        got = d.kv_cache(l)
        W = WINDOWS[l]
        for b in range(batch):
            p = int(pos[b])
            for name in got:
                cache[name][b, :, p] = got[name][b, :, p % W if W else p]

    for step in range(10):
        tok = rng.integers(0, cfg["vocab_size"], batch).astype(np.uint32)
        d.step(stream, dev.upload(tok), logits)
        stream.sync()
        hook = force_rows if kv_cache == "turboquant" else None
        want = ref.step(tok.astype(np.int64), cache_hook=hook)
        want_x = exact.step(tok.astype(np.int64), cache_hook=hook)
        want_32 = exact32.step(tok.astype(np.int64), cache_hook=hook)
        assert_decoder_logits(logits.read(), want, want_x, want_32, f"{kv_cache} B={batch} step {step}")
    # the windowed layers' caches hold W slots
    assert d.kv_cache(1)["k_codes" if kv_cache == "turboquant" else "k"].shape[2] == 5
    if kv_cache == "fp16":
        # the ring of layer 2 holds the last 3 positions' K rows, slot p % 3
        got = d.kv_cache(2)["k"]
        for b in range(batch):
            last = start[b] + 9
            for p in range(last - 2, last + 1):
                assert rel_l2(got[b, :, p % 3], ref.caches[2]["k"][b, :, p]) <= 5e-3


def test_window_beyond_max_seq_refused(dev):
    model = make_model(dev, 92)
    with pytest.raises(IronmillError, match="window_size above max_seq_len"):
        build(dev, model, "fp16", [0, CFG["max_seq_len"] + 1, 0])
