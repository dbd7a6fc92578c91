"""GPU parity of the decoder's prefill (imh_decoder_prefill: run_pipeline_inner with
token_count > 1, metal/pipeline.rs:228-1313).

Causal attention makes a prefill of T tokens the same computation as T decode
steps: token t attends to the positions up to its own.  So the oracle
(DecoderReference) steps through the chunk one token at a time and its last
step's logits are the prefill's; afterwards the GPU decoder and the oracle
decode three more tokens from the caches the prefill wrote.  Tolerances as in
the sliding-window decoder test: rel-L2 1e-3 against the oracle on the GPU
upload's weight semantics (weights="exact"), and 1e-3 plus that oracle's own
distance from the reference's CPU path against the latter.  The chunk sizes
cover both projection paths: 2 x 7 = 14 rows (matvec ops) and 2 x 20 = 40 rows
(the GEMM ops, from 32 rows).  With the TurboQuant cache the oracle takes the
code rows the GPU wrote (bit-exact on equal inputs; rounding differences in
the input can move a vector across a codebook boundary).

Sliding-window layers follow the reference's positions (attention.rs:141-163):
token t of a chunk attends to the ring slots [0, min(p + T, W) - T + t + 1).
While the chunk fits the ring's unwritten slots (p + T <= W) that is the last W
positions up to the token's own, the causal window the oracle computes; that is
the case tested here.  Past it the reference's clamp lets the chunk's early
tokens see slots its later tokens rewrote, which no causal oracle reproduces;
the positions themselves are pinned against the reference's formulas in
test_host.py.
"""
import numpy as np
import pytest

import oracle as O
from conftest import rel_l2
from ironmill_amd import IronmillError, ops
from test_gpu_decode import CFG, make_model

pytestmark = pytest.mark.gpu


def build(dev, model, kv_cache, windows=None, cfg=CFG):
    host_layers, dev_layers, emb, fnorm, lm = model
    d = ops.Decoder(dev, kv_cache=kv_cache, window_sizes=windows, **cfg)
    for l, dl in enumerate(dev_layers):
        d.set_layer(l, **{k: v for k, v in dl.items() if not k.startswith("_")})
    d._keep_lm = ops.AffineQuantizedWeight(dev, lm)
    d.set_model(dev.upload(emb), dev.upload(fnorm), d._keep_lm)
    return d


def check(got, ref_logits, exact_logits, what):
    rx, r, spread = rel_l2(got, exact_logits), rel_l2(got, ref_logits), rel_l2(exact_logits, ref_logits)
    print(f"{what}: rel-L2 vs exact {rx:.2e}, vs CPU path {r:.2e} (oracles apart {spread:.2e})", flush=True)
    assert rx <= 1e-3, f"{what}: rel-L2 {rx:.3e} against the exact-weight oracle"
    assert r <= 1e-3 + spread, f"{what}: rel-L2 {r:.3e} against the CPU path"


@pytest.mark.parametrize("kv_cache,T,windows,batch", [
    ("fp16", 7, None, 2),
    ("turboquant", 7, None, 2),
    ("fp16", 20, None, 2),           # 40 rows: the GEMM ops
    ("turboquant", 20, None, 2),
    # sliding-window layers: the chunk fills the rings up to 12 of 12 and 16 slots, the
    # decode steps after it wrap the smaller one
    ("fp16", 7, [0, 16, 12], 2),
    ("turboquant", 7, [0, 16, 12], 2),
    # one sequence: a 7-row chunk, then the decoder's one-row launches
    ("fp16", 7, None, 1),
    ("turboquant", 7, None, 1),
    ("turboquant", 33, None, 1),     # 33 rows: the GEMM ops with one sequence
])
def test_prefill_matches_stepwise_reference(dev, stream, kv_cache, T, windows, batch):
    cfg = dict(CFG, batch=batch)
    model = make_model(dev, 93)
    d = build(dev, model, kv_cache, windows, cfg)
    host_layers, _, emb, fnorm, lm = model
    kw = dict(kv_cache=kv_cache, window_sizes=windows)
    ref = O.DecoderReference(cfg, host_layers, emb, fnorm, lm, **kw)
    exact = O.DecoderReference(cfg, host_layers, emb, fnorm, lm, weights="exact", acc="f64", **kw)
    start = np.array([0, 5] if batch == 2 else [5], np.int32)
    d.reset(stream, start)
    ref.positions = start.copy()
    exact.positions = start.copy()
    rng = np.random.default_rng(T + 100 * batch)
    B, V = batch, cfg["vocab_size"]
    logits = dev.empty((B, V), np.float16)
    chunk = rng.integers(0, V, (B, T)).astype(np.uint32)
    d.prefill(stream, dev.upload(chunk), T, logits)
    stream.sync()
    assert np.array_equal(d.positions(), start + T)

    def force_rows(l, cache, pos):
        got = d.kv_cache(l)
        W = windows[l] if windows else 0
        for b in range(B):
            p = int(pos[b])
            for name in got:
                cache[name][b, :, p] = got[name][b, :, p % W if W else p]

    hook = force_rows if kv_cache == "turboquant" else None
    for t in range(T):
        want = ref.step(chunk[:, t].astype(np.int64), cache_hook=hook)
        want_x = exact.step(chunk[:, t].astype(np.int64), cache_hook=hook)
    check(logits.read(), want, want_x, f"{kv_cache} T={T} prefill")
    for step in range(3):
        tok = rng.integers(0, V, B).astype(np.uint32)
        d.step(stream, dev.upload(tok), logits)
        stream.sync()
        want = ref.step(tok.astype(np.int64), cache_hook=hook)
        want_x = exact.step(tok.astype(np.int64), cache_hook=hook)
        check(logits.read(), want, want_x, f"{kv_cache} T={T} decode {step}")


def test_prefill_errors(dev, stream):
    model = make_model(dev, 94)
    d = build(dev, model, "fp16", [0, 4, 0])
    B, V = CFG["batch"], CFG["vocab_size"]
    logits = dev.empty((B, V), np.float16)
    with pytest.raises(IronmillError, match="window"):
        d.prefill(stream, dev.upload(np.zeros((B, 5), np.uint32)), 5, logits)
    d.reset(stream, np.array([61, 0], np.int32))
    with pytest.raises(IronmillError, match="beyond max_seq_len"):
        d.prefill(stream, dev.upload(np.zeros((B, 4), np.uint32)), 4, logits)
