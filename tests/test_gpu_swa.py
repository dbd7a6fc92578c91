"""GPU parity of sliding-window attention layers in the decode step.

The decoder keeps a windowed layer's cache as a ring of W slots (the buffer
stride, write position and attention bound of attention.rs:141-163 and
turboquant/cache.rs:382-400); the oracle (DecoderReference with window_sizes)
keeps a linear cache and attends to the last W positions of each sequence, the
definition the ring implements.  Layers 1 and 2 use windows of 5 and 3
positions, layer 0 full attention; two sequences start at positions 0 and 9
and decode 10 tokens, so both rings wrap several times.  At every step the
logits must stay within the north star's rel-L2 1e-3 of the oracle on the GPU
upload's weight semantics (weights="exact": (q - z16) * s16, f64 sums), and
within 1e-3 plus that oracle's own distance from the reference's CPU path
(f16-dequantized weights) of the latter: this model's logits move by ~1e-3
between those two weight semantics alone (measured 0.8-1.2e-3 per step, with
and without windows), so 1e-3 against the CPU path is not a bound the
semantics allow here.  With the TurboQuant cache
the oracle takes the code rows the GPU wrote (slot p % W of a windowed layer
holds position p), as in the full-attention decoder test: the cache write is
bit-exact on equal inputs, and rounding differences in its input can move a
vector across a codebook boundary.
"""
import numpy as np
import pytest

import oracle as O
from conftest import rel_l2
from ironmill_amd import IronmillError, ops
from test_gpu_decode import CFG, make_model

pytestmark = pytest.mark.gpu

WINDOWS = [0, 5, 3]


def build(dev, model, kv_cache, windows):
    host_layers, dev_layers, emb, fnorm, lm = model
    d = ops.Decoder(dev, kv_cache=kv_cache, window_sizes=windows, **CFG)
    for l, dl in enumerate(dev_layers):
        d.set_layer(l, **{k: v for k, v in dl.items() if not k.startswith("_")})
    d._keep_lm = ops.AffineQuantizedWeight(dev, lm)
    d.set_model(dev.upload(emb), dev.upload(fnorm), d._keep_lm)
    return d


@pytest.mark.parametrize("kv_cache", ["fp16", "turboquant"])
def test_decoder_sliding_window_matches_reference(dev, stream, kv_cache):
    model = make_model(dev, 91)
    d = build(dev, model, kv_cache, WINDOWS)
    host_layers, _, emb, fnorm, lm = model
    ref = O.DecoderReference(CFG, host_layers, emb, fnorm, lm, kv_cache=kv_cache, window_sizes=WINDOWS)
    exact = O.DecoderReference(CFG, host_layers, emb, fnorm, lm, kv_cache=kv_cache, window_sizes=WINDOWS,
                               weights="exact", acc="f64")
    start = np.array([0, 9], np.int32)
    d.reset(stream, start)
    ref.positions = start.copy()
    exact.positions = start.copy()
    rng = np.random.default_rng(6)
    logits = dev.empty((CFG["batch"], CFG["vocab_size"]), np.float16)

    def force_rows(l, cache, pos):
        got = d.kv_cache(l)
        W = WINDOWS[l]
        for b in range(CFG["batch"]):
            p = int(pos[b])
            for name in got:
                cache[name][b, :, p] = got[name][b, :, p % W if W else p]

    for step in range(10):
        tok = rng.integers(0, CFG["vocab_size"], CFG["batch"]).astype(np.uint32)
        d.step(stream, dev.upload(tok), logits)
        stream.sync()
        hook = force_rows if kv_cache == "turboquant" else None
        want = ref.step(tok.astype(np.int64), cache_hook=hook)
        want_x = exact.step(tok.astype(np.int64), cache_hook=hook)
        got = logits.read()
        rx, r, spread = rel_l2(got, want_x), rel_l2(got, want), rel_l2(want_x, want)
        print(f"step {step}: rel-L2 vs exact {rx:.2e}, vs CPU path {r:.2e} (oracles apart {spread:.2e})")
        assert rx <= 1e-3, f"{kv_cache} step {step}: logits rel-L2 {rx:.3e} against the exact-weight oracle"
        assert r <= 1e-3 + spread, f"{kv_cache} step {step}: logits rel-L2 {r:.3e} against the CPU path"
    # the windowed layers' caches hold W slots
    assert d.kv_cache(1)["k_codes" if kv_cache == "turboquant" else "k"].shape[2] == 5
    if kv_cache == "fp16":
        # the ring of layer 2 holds the last 3 positions' K rows, slot p % 3
        got = d.kv_cache(2)["k"]
        for b in range(CFG["batch"]):
            last = start[b] + 9
            for p in range(last - 2, last + 1):
                assert rel_l2(got[b, :, p % 3], ref.caches[2]["k"][b, :, p]) <= 5e-3


def test_window_beyond_max_seq_refused(dev):
    model = make_model(dev, 92)
    with pytest.raises(IronmillError, match="window_size above max_seq_len"):
        build(dev, model, "fp16", [0, CFG["max_seq_len"] + 1, 0])
