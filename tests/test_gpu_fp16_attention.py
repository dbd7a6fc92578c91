"""GPU parity of the FP16 KV cache ops (the non-quantized comparator of the
TurboQuant path) against the CPU oracle.

* kv_scatter (kv_scatter.metal:20-45): cache rows == projections, bit for bit,
  with the ring-buffer wrap at max_seq_len;
* attention (fused_sdpa.metal:52-251 + flash_decode.metal:25-215) == the
  oracle's f64 cpu_attention (inference.rs:222-280) within rel-L2 <= 1e-3 and
  max-abs <= 2e-2, for single/split KV ranges, GQA 1/2/4, ragged and empty
  sequences, causal multi-token queries, and the 32k-context configuration;
* one position: the softmax weight is exactly 1, so the output is V bit for bit.
"""
import math

import numpy as np
import pytest

import oracle as O
from conftest import assert_close
from ironmill_amd import IronmillError, ops

pytestmark = pytest.mark.gpu

D = 128
SCALE = 1.0 / math.sqrt(D)


def kv_data(batch, tokens, nkv, seed):
    """K/V fp16 N(0,1) with 4 seeded outlier channels per head scaled x10."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, tokens, nkv, D)).astype(np.float32)
    for h in range(nkv):
        ch = rng.choice(D, 4, replace=False)
        x[:, :, h, ch] *= 10.0
    return x.astype(np.float16)


def fill_cache(dev, stream, batch, nkv, max_seq, ctx, seed):
    cache = ops.Fp16KvCache(dev, batch, nkv, D, max_seq)
    cache.zero(stream)
    if ctx:
        k, v = kv_data(batch, ctx, nkv, seed), kv_data(batch, ctx, nkv, seed + 1)
        ops.encode_kv_scatter(stream, cache, dev.upload(k), ctx, 0, True)
        ops.encode_kv_scatter(stream, cache, dev.upload(v), ctx, 0, False)
    stream.sync()
    return cache


def run_attention(dev, stream, cache, q16, nh, seq_len, seq_lens=None, num_splits=0):
    token_count = 1 if q16.ndim == 3 else q16.shape[1]
    out = dev.empty(q16.shape, np.float16)
    sl = dev.upload(np.asarray(seq_lens, np.int32)) if seq_lens is not None else None
    ops.encode_fp16_attention(stream, cache, dev.upload(q16), nh, seq_len, out, token_count=token_count,
                              attn_scale=SCALE, seq_lens=sl, num_splits=num_splits)
    stream.sync()
    return out.read()


@pytest.mark.parametrize("is_k", [True, False])
def test_scatter_bit_exact(dev, stream, is_k):
    batch, tokens, nkv, max_seq = 3, 5, 8, 64
    proj = kv_data(batch, tokens, nkv, seed=7 + is_k)
    positions = np.array([0, 17, 62], np.int32)  # the last one wraps around (% max_seq)
    cache = ops.Fp16KvCache(dev, batch, nkv, D, max_seq)
    cache.zero(stream)
    ops.encode_kv_scatter(stream, cache, dev.upload(proj), tokens, 0, is_k, positions=dev.upload(positions))
    stream.sync()
    got = (cache.k if is_k else cache.v).read()
    other = (cache.v if is_k else cache.k).read()
    ref = np.zeros_like(got)
    for b in range(batch):
        for t in range(tokens):
            ref[b, :, (positions[b] + t) % max_seq] = proj[b, t]
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    assert not other.view(np.uint16).any()


@pytest.mark.parametrize("nh,nkv", [(32, 8), (16, 8), (8, 8)])
@pytest.mark.parametrize("num_splits", [0, 1, 7])
def test_attention_matches_oracle(dev, stream, nh, nkv, num_splits):
    batch, ctx, max_seq = 2, 300, 512
    cache = fill_cache(dev, stream, batch, nkv, max_seq, ctx, seed=100 + nh)
    q16 = np.random.default_rng(5).standard_normal((batch, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, cache, q16, nh, ctx, num_splits=num_splits)
    ref = O.fp16_attention(q16, cache.k.read(), cache.v.read(), ctx, SCALE, nthreads=8)
    assert_close(got, ref, what=f"fp16 attention nh={nh} nkv={nkv} splits={num_splits}")


@pytest.mark.parametrize("nh,nkv", [(32, 8), (16, 8), (8, 8)])
@pytest.mark.parametrize("tokens", [2, 7])
def test_causal_multi_token(dev, stream, nh, nkv, tokens):
    batch, ctx, max_seq = 2, 200, 256
    cache = fill_cache(dev, stream, batch, nkv, max_seq, ctx, seed=40 + tokens)
    q16 = np.random.default_rng(tokens).standard_normal((batch, tokens, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, cache, q16, nh, ctx, num_splits=3)
    ref = O.fp16_attention(q16, cache.k.read(), cache.v.read(), ctx, SCALE, nthreads=8)
    assert_close(got, ref, what=f"causal T={tokens} nh={nh}")


def test_split_and_single_pass_agree(dev, stream):
    cache = fill_cache(dev, stream, 1, 8, 4096, 4000, seed=3)
    q16 = np.random.default_rng(6).standard_normal((1, 32, D)).astype(np.float16)
    a = run_attention(dev, stream, cache, q16, 32, 4000, num_splits=1).astype(np.float32)
    b = run_attention(dev, stream, cache, q16, 32, 4000, num_splits=40).astype(np.float32)
    assert_close(a, b, rel=2e-3, max_abs=2e-3, what="split vs single")


@pytest.mark.parametrize("bound", [400, 0])  # 0: the splits span max_seq_len
def test_ragged_and_empty_sequences(dev, stream, bound):
    batch, nkv, nh, max_seq = 4, 8, 32, 512
    cache = fill_cache(dev, stream, batch, nkv, max_seq, 400, seed=9)
    lens = np.array([400, 1, 0, 77], np.int32)
    q16 = np.random.default_rng(8).standard_normal((batch, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, cache, q16, nh, bound, seq_lens=lens)
    ref = O.fp16_attention(q16, cache.k.read(), cache.v.read(), 400, SCALE, seq_lens=lens, nthreads=8)
    assert_close(got, ref, what="ragged")
    assert np.array_equal(got[2].view(np.uint16), np.zeros((nh, D), np.uint16))  # empty -> 0


def test_single_position_returns_value(dev, stream):
    """seq_len 1: the weight is exactly 1, so out is V bit for bit (closed form)."""
    cache = fill_cache(dev, stream, 2, 8, 64, 1, seed=11)
    q16 = np.random.default_rng(1).standard_normal((2, 32, D)).astype(np.float16)
    got = run_attention(dev, stream, cache, q16, 32, 1)
    v = cache.v.read()
    for h in range(32):
        assert np.array_equal(got[:, h].view(np.uint16), v[:, h // 4, 0].view(np.uint16)), h


@pytest.mark.parametrize("batch,ctx", [(1, 32768), (16, 2048)])
def test_attention_full_size(dev, stream, batch, ctx):
    nkv, nh = 8, 32
    cache = fill_cache(dev, stream, batch, nkv, ctx, ctx, seed=ctx + batch)
    q16 = np.random.default_rng(12).standard_normal((batch, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, cache, q16, nh, ctx)
    ref = O.fp16_attention(q16, cache.k.read(), cache.v.read(), ctx, SCALE, nthreads=8)
    assert_close(got, ref, what=f"full size B={batch} ctx={ctx}")


def test_decode_step_write_then_attend(dev, stream):
    batch, nkv, nh, max_seq, pos = 2, 8, 32, 256, 150
    cache = fill_cache(dev, stream, batch, nkv, max_seq, pos, seed=21)
    k1, v1 = kv_data(batch, 1, nkv, 22), kv_data(batch, 1, nkv, 23)
    q16 = np.random.default_rng(24).standard_normal((batch, nh, D)).astype(np.float16)
    out = dev.empty((batch, nh, D), np.float16)
    ops.encode_fp16_kv_cache_and_attention(stream, cache, dev.upload(k1), dev.upload(v1), dev.upload(q16),
                                           nh, pos, out)
    stream.sync()
    kc, vc = cache.k.read(), cache.v.read()
    assert np.array_equal(kc[:, :, pos].view(np.uint16), k1[:, 0].view(np.uint16))
    assert np.array_equal(vc[:, :, pos].view(np.uint16), v1[:, 0].view(np.uint16))
    ref = O.fp16_attention(q16, kc, vc, pos + 1, SCALE, nthreads=8)
    assert_close(out.read(), ref, what="fp16 decode step")


def test_attention_error_paths(dev, stream):
    cache = ops.Fp16KvCache(dev, 1, 8, D, 64)
    q = dev.empty((1, 32, D), np.float16)
    out = dev.empty((1, 32, D), np.float16)
    with pytest.raises(IronmillError, match="exceeds max_seq_len"):
        ops.encode_fp16_attention(stream, cache, q, 32, 65, out)
    with pytest.raises(IronmillError, match="multiple of num_kv_heads"):
        ops.encode_fp16_attention(stream, cache, q, 30, 10, out)
    with pytest.raises(IronmillError, match="not built"):
        ops.encode_fp16_attention(stream, cache, q, 64, 10, out)
    with pytest.raises(IronmillError, match="token_count exceeds seq_len"):
        ops.encode_fp16_attention(stream, cache, q, 32, 1, out, token_count=2)
    with pytest.raises(IronmillError, match="exceeds max_seq_len"):
        ops.encode_fp16_kv_cache_and_attention(stream, cache, q, q, q, 32, 64, out)
    with pytest.raises(IronmillError, match="built for head_dim 128"):
        ops.encode_fp16_attention(stream, ops.Fp16KvCache(dev, 1, 8, 64, 64), q, 32, 1, out)
