"""GPU parity of the TurboQuant INT8 KV cache ops against the CPU oracle.

* tables made by the library == the oracle's restatement of
  MetalTurboQuantModel::new (mod.rs:221-287), bit for bit;
* cache-write codes, scales and residual norms == oracle, bit for bit
  (turboquant.metal:52-170 in the fixed f32 order both sides implement);
* decode attention == oracle's f64 dequantize-then-compute attention within
  rel-L2 <= 1e-3 and max-abs <= 2e-2, for single/split KV ranges, ragged and
  empty sequences, GQA 1/2/4, and the 32k-context configuration.
"""
import math

import numpy as np
import pytest

import oracle as O
from conftest import assert_close
from ironmill_amd import IronmillError, ops

pytestmark = pytest.mark.gpu

D = 128


@pytest.fixture(scope="module")
def tq(dev):
    return ops.TurboQuantModel(dev, D, 8, 42)


@pytest.fixture(scope="module")
def tables():
    return O.TQTables(D, 8, 42)


def kv_data(batch, tokens, nkv, seed, outliers=True):
    """K/V fp16 N(0,1) with 4 seeded outlier channels per head scaled x10."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, tokens, nkv, D)).astype(np.float32)
    for h in range(nkv if outliers else 0):
        ch = rng.choice(D, 4, replace=False)
        x[:, :, h, ch] *= 10.0
    return x.astype(np.float16)


def test_tables_match_oracle(tq, tables):
    t = tq.tables()
    for name in ("signs", "k_codebook", "k_bounds", "v_codebook", "v_bounds"):
        ref = getattr(tables, name)
        assert np.array_equal(t[name].view(np.uint32), ref.view(np.uint32)), name
    assert np.array_equal(t["qjl"].view(np.uint32), tables.qjl.view(np.uint32))


@pytest.mark.parametrize("is_k", [True, False])
def test_cache_write_bit_exact(dev, stream, tq, tables, is_k):
    batch, tokens, nkv, max_seq = 3, 5, 8, 64
    kv = kv_data(batch, tokens, nkv, seed=7 + is_k)
    positions = np.array([0, 17, 62], np.int32)  # the last one wraps around (% max_seq)
    cache = ops.TurboQuantKvCache(dev, batch, nkv, D, max_seq)
    cache.zero(stream)
    kd, pd = dev.upload(kv), dev.upload(positions)
    ops.encode_turboquant_cache_write(stream, tq, cache, kd, tokens, 0, is_k, positions=pd)
    stream.sync()
    codes_ref, sc_ref, rn_ref = O.tq_cache_write(kv, tables, is_k, max_seq, positions=positions)
    codes = (cache.k_codes if is_k else cache.v_codes).read()
    scales = (cache.k_scales if is_k else cache.v_scales).read()
    assert np.array_equal(codes, codes_ref)
    assert np.array_equal(scales.view(np.uint32), sc_ref.view(np.uint32))
    if is_k:
        assert np.array_equal(cache.k_r_norms.read().view(np.uint32), rn_ref.view(np.uint32))


def test_cache_write_kv_one_launch_bit_exact(dev, stream, tq, tables):
    """K and V written by the one-launch entry point == the oracle's writes, bit for bit."""
    batch, tokens, nkv, max_seq = 2, 7, 8, 32
    k, v = kv_data(batch, tokens, nkv, seed=31), kv_data(batch, tokens, nkv, seed=32)
    positions = np.array([3, 29], np.int32)   # the second wraps around
    cache = ops.TurboQuantKvCache(dev, batch, nkv, D, max_seq)
    cache.zero(stream)
    ops.encode_turboquant_cache_write_kv(stream, tq, cache, dev.upload(k), dev.upload(v), tokens, 0,
                                         positions=dev.upload(positions))
    stream.sync()
    kc, ks, kr = O.tq_cache_write(k, tables, True, max_seq, positions=positions)
    vc, vs, _ = O.tq_cache_write(v, tables, False, max_seq, positions=positions)
    assert np.array_equal(cache.k_codes.read(), kc) and np.array_equal(cache.v_codes.read(), vc)
    assert np.array_equal(cache.k_scales.read().view(np.uint32), ks.view(np.uint32))
    assert np.array_equal(cache.v_scales.read().view(np.uint32), vs.view(np.uint32))
    assert np.array_equal(cache.k_r_norms.read().view(np.uint32), kr.view(np.uint32))


def test_cache_write_unsorted_boundaries_scan(dev, stream):
    """Caller tables whose boundaries are not sorted take the linear scan, which keeps the
    reference's "last boundary <= u" rule (turboquant.metal:118-124) bit for bit."""
    tabs = O.TQTables(D, 8, 7)
    rng = np.random.default_rng(3)
    for bd in (tabs.k_bounds, tabs.v_bounds):
        i = rng.choice(bd.size - 8, 4, replace=False) + 4
        bd[i], bd[i + 3] = bd[i + 3].copy(), bd[i].copy()   # local disorder
    host = dict(signs=tabs.signs, k_codebook=tabs.k_codebook, k_bounds=tabs.k_bounds,
                v_codebook=tabs.v_codebook, v_bounds=tabs.v_bounds, qjl=tabs.qjl)
    tq2 = ops.TurboQuantModel(dev, D, 8, host_tables=host)
    kv = kv_data(1, 40, 8, seed=5)
    cache = ops.TurboQuantKvCache(dev, 1, 8, D, 64)
    cache.zero(stream)
    ops.encode_turboquant_cache_write_kv(stream, tq2, cache, dev.upload(kv), dev.upload(kv), 40, 0)
    stream.sync()
    kc, _, _ = O.tq_cache_write(kv, tabs, True, 64)
    vc, _, _ = O.tq_cache_write(kv, tabs, False, 64)
    assert np.array_equal(cache.k_codes.read(), kc) and np.array_equal(cache.v_codes.read(), vc)


def fill_cache(dev, stream, tq, batch, nkv, max_seq, ctx, seed, outliers=True):
    cache = ops.TurboQuantKvCache(dev, batch, nkv, D, max_seq)
    cache.zero(stream)
    k = kv_data(batch, ctx, nkv, seed, outliers)
    v = kv_data(batch, ctx, nkv, seed + 1, outliers)
    kd, vd = dev.upload(k), dev.upload(v)
    ops.encode_turboquant_cache_write(stream, tq, cache, kd, ctx, 0, True)
    ops.encode_turboquant_cache_write(stream, tq, cache, vd, ctx, 0, False)
    stream.sync()
    return cache


def read_cache(cache):
    return (cache.k_codes.read(), cache.v_codes.read(), cache.k_scales.read(), cache.v_scales.read(),
            cache.k_r_norms.read())


def run_attention(dev, stream, tq, cache, q16, nh, seq_len, seq_lens=None, num_splits=0):
    qd = dev.upload(q16)
    out = dev.empty(q16.shape, np.float16)
    sl = dev.upload(np.asarray(seq_lens, np.int32)) if seq_lens is not None else None
    ops.encode_turboquant_attention(stream, tq, cache, qd, nh, seq_len, out, 1.0 / math.sqrt(D),
                                    seq_lens=sl, num_splits=num_splits)
    stream.sync()
    return out.read()


@pytest.mark.parametrize("nh,nkv", [(32, 8), (16, 8), (8, 8)])
@pytest.mark.parametrize("num_splits", [0, 1, 7])
def test_attention_matches_oracle(dev, stream, tq, tables, nh, nkv, num_splits):
    batch, ctx, max_seq = 2, 300, 512
    cache = fill_cache(dev, stream, tq, batch, nkv, max_seq, ctx, seed=100 + nh)
    q16 = np.random.default_rng(5).standard_normal((batch, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, tq, cache, q16, nh, ctx, num_splits=num_splits)
    kc, vc, ks, vs, kr = read_cache(cache)
    ref = O.tq_attention(q16, tables, kc, vc, ks, vs, kr, ctx, 1.0 / math.sqrt(D), nthreads=8)
    assert_close(got, ref, what=f"attention nh={nh} nkv={nkv} splits={num_splits}")


def test_split_and_single_pass_agree(dev, stream, tq):
    cache = fill_cache(dev, stream, tq, 1, 8, 4096, 4000, seed=3)
    q16 = np.random.default_rng(6).standard_normal((1, 32, D)).astype(np.float16)
    a = run_attention(dev, stream, tq, cache, q16, 32, 4000, num_splits=1).astype(np.float32)
    b = run_attention(dev, stream, tq, cache, q16, 32, 4000, num_splits=40).astype(np.float32)
    assert_close(a, b, rel=2e-3, max_abs=2e-3, what="split vs single")


@pytest.mark.parametrize("bound", [400, 0])  # 0: the splits span max_seq_len
def test_ragged_and_empty_sequences(dev, stream, tq, tables, bound):
    batch, nkv, nh, max_seq = 4, 8, 32, 512
    cache = fill_cache(dev, stream, tq, batch, nkv, max_seq, 400, seed=9)
    lens = np.array([400, 1, 0, 77], np.int32)
    q16 = np.random.default_rng(8).standard_normal((batch, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, tq, cache, q16, nh, bound, seq_lens=lens)
    kc, vc, ks, vs, kr = read_cache(cache)
    ref = O.tq_attention(q16, tables, kc, vc, ks, vs, kr, 400, 1.0 / math.sqrt(D), seq_lens=lens,
                         nthreads=8)
    assert_close(got, ref, what="ragged")
    assert np.array_equal(got[2].view(np.uint16), np.zeros((nh, D), np.uint16))  # empty -> 0


def test_single_position_returns_rotated_value(dev, stream, tq, tables):
    """seq_len 1: softmax weight is 1, so out = R (vcb[c] * v_scale) (closed form).  The
    codebook value and the weight times the V scale enter the matrix cores as f16, so the
    closed form holds to ~2^-11 relative, inside the north-star bound used here."""
    cache = fill_cache(dev, stream, tq, 1, 8, 64, 1, seed=11)
    q16 = np.random.default_rng(1).standard_normal((1, 32, D)).astype(np.float16)
    got = run_attention(dev, stream, tq, cache, q16, 32, 1)
    vc, vs = cache.v_codes.read(), cache.v_scales.read()
    for h in range(32):
        kvh = h // 4
        v = tables.v_codebook[vc[0, kvh, 0]].astype(np.float64) * vs[0, kvh, 0]
        ref = O.hadamard_rotate(v.astype(np.float32), tables.signs)
        assert_close(got[0, h], ref, what=f"head {h}")


@pytest.mark.parametrize("batch,ctx", [(1, 32768), (16, 2048)])
def test_attention_full_size(dev, stream, tq, tables, batch, ctx):
    nkv, nh = 8, 32
    cache = fill_cache(dev, stream, tq, batch, nkv, ctx, ctx, seed=ctx + batch)
    q16 = np.random.default_rng(12).standard_normal((batch, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, tq, cache, q16, nh, ctx)
    kc, vc, ks, vs, kr = read_cache(cache)
    ref = O.tq_attention(q16, tables, kc, vc, ks, vs, kr, ctx, 1.0 / math.sqrt(D), nthreads=8)
    assert_close(got, ref, what=f"full size B={batch} ctx={ctx}")


def fill_cache_blocks(dev, stream, tq, batch, nkv, ctx, block, seed):
    """A cache of ctx positions per sequence written block by block (configs[2] data, one
    seeded block of K/V rows per sequence, repeated every `block` positions)."""
    cache = ops.TurboQuantKvCache(dev, batch, nkv, D, ctx)
    cache.zero(stream)
    k = kv_data(batch, block, nkv, seed)
    v = kv_data(batch, block, nkv, seed + 1)
    kd, vd = dev.upload(k), dev.upload(v)
    for base in range(0, ctx, block):
        ops.encode_turboquant_cache_write_kv(stream, tq, cache, kd, vd, min(block, ctx - base), base)
    stream.sync()
    return cache


@pytest.mark.parametrize("batch,ctx", [(1, 2048), (8, 2048), (8, 8192), (16, 8192), (8, 32768), (16, 32768)])
def test_attention_benchmarked_shapes(dev, stream, tq, tables, batch, ctx):
    """Every (batch, context) of configs[2] that the benchmark reports beyond the cases
    above: all rows against the oracle, and the automatic split against one split (the
    split-combine identity, to f32 rounding)."""
    nkv, nh = 8, 32
    print(f"tq attention B={batch} ctx={ctx}", flush=True)
    cache = fill_cache_blocks(dev, stream, tq, batch, nkv, ctx, min(ctx, 4096), seed=ctx // 7 + batch)
    q16 = np.random.default_rng(14 + batch).standard_normal((batch, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, tq, cache, q16, nh, ctx)
    one = run_attention(dev, stream, tq, cache, q16, nh, ctx, num_splits=1)
    kc, vc, ks, vs, kr = read_cache(cache)
    ref = O.tq_attention(q16, tables, kc, vc, ks, vs, kr, ctx, 1.0 / math.sqrt(D), nthreads=16)
    assert_close(got, ref, what=f"B={batch} ctx={ctx}")
    assert_close(one, ref, what=f"B={batch} ctx={ctx}, one split")
    assert_close(got.astype(np.float32), one.astype(np.float32), rel=2e-3, max_abs=2e-3, what="split vs single")


def test_attention_long_context_plain_normal(dev, stream, tq, tables):
    """Plain N(0,1) K/V at 30000 positions: the weights are nearly uniform, so the output
    shrinks as 1/sqrt(positions) while a rounding bias of the V codebook does not.  With the
    codebook in f16 alone this case gives rel-L2 1.9e-3 (computed on the CPU with the rounded
    codebook); the hi + lo codebook keeps it near the f16 weight rounding (~2e-4)."""
    nkv, nh, ctx = 8, 32, 30000
    cache = fill_cache(dev, stream, tq, 1, nkv, ctx, ctx, seed=77, outliers=False)
    q16 = np.random.default_rng(13).standard_normal((1, nh, D)).astype(np.float16)
    got = run_attention(dev, stream, tq, cache, q16, nh, ctx)
    kc, vc, ks, vs, kr = read_cache(cache)
    ref = O.tq_attention(q16, tables, kc, vc, ks, vs, kr, ctx, 1.0 / math.sqrt(D), nthreads=8)
    assert_close(got, ref, rel=5e-4, what="plain N(0,1) K/V, 30000 positions")


@pytest.mark.parametrize("batch,nh,pos,max_seq", [(2, 32, 150, 256), (1, 8, 0, 64), (3, 16, 4095, 8192),
                                                  (1, 32, 8191, 8192)])
def test_decode_step_write_then_attend(dev, stream, tq, tables, batch, nh, pos, max_seq):
    """encode_kv_cache_and_attention: the token's K / V are written in the attention launch
    (one extra workgroup per kv head and sequence) -- codes, scales and residual norms at row
    pos bit-exact with the oracle's write, every other row untouched, and the output equal to
    the oracle's attention over [0, pos] of the written cache.  Covers the first position (no
    other split has work), many splits, GQA 1 / 2 / 4 and the cache's last row."""
    nkv = 8
    if pos:
        cache = fill_cache(dev, stream, tq, batch, nkv, max_seq, pos, seed=21 + pos)
    else:
        cache = ops.TurboQuantKvCache(dev, batch, nkv, D, max_seq)
        cache.zero(stream)
        stream.sync()
    before = read_cache(cache)
    k1, v1 = kv_data(batch, 1, nkv, 22), kv_data(batch, 1, nkv, 23)
    q16 = np.random.default_rng(24).standard_normal((batch, nh, D)).astype(np.float16)
    out = dev.empty((batch, nh, D), np.float16)
    ops.encode_kv_cache_and_attention(stream, tq, cache, dev.upload(k1), dev.upload(v1),
                                      dev.upload(q16), nh, pos, out)
    stream.sync()
    kc, vc, ks, vs, kr = read_cache(cache)
    kc1, ks1, kr1 = O.tq_cache_write(k1, tables, True, 1)
    vc1, vs1, _ = O.tq_cache_write(v1, tables, False, 1)
    assert np.array_equal(kc[:, :, pos], kc1[:, :, 0]) and np.array_equal(vc[:, :, pos], vc1[:, :, 0])
    for got, ref in ((ks, ks1), (kr, kr1), (vs, vs1)):
        assert np.array_equal(got[:, :, pos].view(np.uint32), ref[:, :, 0].view(np.uint32))
    other = np.arange(max_seq) != pos
    for got, old in zip((kc, vc, ks, vs, kr), before):
        assert np.array_equal(got[:, :, other], old[:, :, other])
    ref = O.tq_attention(q16, tables, kc, vc, ks, vs, kr, pos + 1, 1.0 / math.sqrt(D), nthreads=8)
    # the token's position is combined in f32 (no f16 weight), the rest as in the plain
    # attention (~3e-4)
    assert_close(out.read(), ref, rel=5e-4, what=f"decode step B={batch} nh={nh} pos={pos}")


@pytest.mark.parametrize("nh,tokens,ragged", [(32, 5, False), (16, 3, True), (8, 7, False)])
def test_attention_multi_token_causal(dev, stream, tq, tables, nh, tokens, ragged):
    """Prefill form (turboquant.metal:268): token t of sequence b attends to positions
    < L_b - T + t + 1; each token equals the one-token oracle at that length.  Ragged:
    per-sequence lengths, one shorter than T (its early tokens see nothing -> 0)."""
    nkv, batch, max_seq = 8, 2, 1024
    cache = fill_cache(dev, stream, tq, batch, nkv, max_seq, 700, seed=61 + tokens)
    q16 = np.random.default_rng(62).standard_normal((batch, tokens, nh, D)).astype(np.float16)
    out = dev.empty((batch, tokens, nh, D), np.float16)
    lens = np.array([700, tokens - 2 if ragged else 433], np.int32)
    ops.encode_turboquant_attention(stream, tq, cache, dev.upload(q16), nh, 0, out, 1.0 / math.sqrt(D),
                                    seq_lens=dev.upload(lens), token_count=tokens)
    stream.sync()
    got = out.read()
    kc, vc, ks, vs, kr = read_cache(cache)
    for t in range(tokens):
        lt = np.maximum(lens - tokens + t + 1, 0).astype(np.int32)
        ref = O.tq_attention(q16[:, t], tables, kc, vc, ks, vs, kr, max_seq, 1.0 / math.sqrt(D),
                             seq_lens=lt, nthreads=8)
        for bb in range(batch):
            if lt[bb] == 0:
                assert not got[bb, t].astype(np.float32).any()
            else:
                assert_close(got[bb, t], ref[bb], rel=5e-4, what=f"token {t} of seq {bb} (len {lt[bb]})")


@pytest.mark.parametrize("nh,tokens,num_splits,lens", [
    (32, 64, 0, (900, 283)),   # GQA 4: 16 token blocks, automatic splits
    (32, 37, 1, (900, 283)),   # a partial last block, normalised in the kernel
    (16, 20, 3, (900, 283)),   # GQA 2, merged by the combine
    (8, 33, 1, (900, 40)),     # GQA 1 (16 tokens per block), a range shorter than the chunk
    (32, 16, 0, None),         # one seq_len for both sequences
])
def test_attention_prefill_token_blocks(dev, stream, tq, tables, nh, tokens, num_splits, lens):
    """The token-block prefill kernel (16 / GQA tokens x the GQA heads per workgroup, each
    row with its own causal bound): every token equals the one-token oracle at its own
    length (turboquant.metal:268), for full and partial blocks, one split and several."""
    nkv, batch, max_seq = 8, 2, 1024
    cache = fill_cache(dev, stream, tq, batch, nkv, max_seq, 900, seed=81 + tokens)
    q16 = np.random.default_rng(82 + tokens).standard_normal((batch, tokens, nh, D)).astype(np.float16)
    out = dev.empty((batch, tokens, nh, D), np.float16)
    if lens is None:
        seq_len, sl, lens = 500, None, np.array([500, 500], np.int32)
    else:
        lens = np.array(lens, np.int32)
        seq_len, sl = 0, dev.upload(lens)
    ops.encode_turboquant_attention(stream, tq, cache, dev.upload(q16), nh, seq_len, out, 1.0 / math.sqrt(D),
                                    seq_lens=sl, num_splits=num_splits, token_count=tokens)
    stream.sync()
    got = out.read()
    kc, vc, ks, vs, kr = read_cache(cache)
    for t in range(tokens):
        lt = np.maximum(lens - tokens + t + 1, 0).astype(np.int32)
        ref = O.tq_attention(q16[:, t], tables, kc, vc, ks, vs, kr, max_seq, 1.0 / math.sqrt(D),
                             seq_lens=lt, nthreads=8)
        assert_close(got[:, t], ref, rel=5e-4, what=f"token {t} (lengths {lt.tolist()})")


def test_graph_replay_after_scratch_growth(dev, tq):
    """A graph keeps addressing the stream scratch it was captured with: a larger eager op
    that grows the scratch afterwards must not free it (the replay equals the eager run,
    bit for bit), and the graph refuses a stream other than the capturing one."""
    s1, s2 = dev.stream(), dev.stream()
    small = fill_cache(dev, s1, tq, 1, 8, 1024, 1000, seed=71)
    big = fill_cache(dev, s1, tq, 4, 8, 8192, 8192, seed=72)
    q_small = dev.upload(np.random.default_rng(73).standard_normal((1, 32, D)).astype(np.float16))
    q_big = dev.upload(np.random.default_rng(74).standard_normal((4, 32, D)).astype(np.float16))
    eager, replay = dev.empty((1, 32, D), np.float16), dev.empty((1, 32, D), np.float16)
    out_big = dev.empty((4, 32, D), np.float16)
    ops.encode_turboquant_attention(s1, tq, small, q_small, 32, 1000, eager, num_splits=8)
    s1.sync()
    graph = s1.capture(lambda: ops.encode_turboquant_attention(s1, tq, small, q_small, 32, 1000, replay,
                                                               num_splits=8))
    # grows the split-partial and counter slots past the captured blocks
    ops.encode_turboquant_attention(s1, tq, big, q_big, 32, 8192, out_big, num_splits=64)
    for _ in range(3):
        graph.launch(s1)
        s1.sync()
        assert np.array_equal(replay.read().view(np.uint16), eager.read().view(np.uint16))
    with pytest.raises(IronmillError, match="captured on"):
        graph.launch(s2)
    graph.close()


def test_attention_error_paths(dev, stream, tq):
    cache = ops.TurboQuantKvCache(dev, 1, 8, D, 64)
    q = dev.empty((1, 32, D), np.float16)
    out = dev.empty((1, 32, D), np.float16)
    with pytest.raises(IronmillError, match="exceeds max_seq_len"):
        ops.encode_turboquant_attention(stream, tq, cache, q, 32, 65, out)
    with pytest.raises(IronmillError, match="multiple of num_kv_heads"):
        ops.encode_turboquant_attention(stream, tq, cache, q, 30, 10, out)
    with pytest.raises(IronmillError, match="beyond max_seq_len"):
        ops.encode_kv_cache_and_attention(stream, tq, cache, q, q, q, 32, 64, out)
    with pytest.raises(IronmillError, match="power of two"):
        ops.TurboQuantModel(dev, 96, 8, 42)
    with pytest.raises(IronmillError, match="built for head_dim 128"):
        ops.TurboQuantModel(dev, 64, 8, 42)
