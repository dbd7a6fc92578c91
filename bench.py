#!/usr/bin/env python3
"""Benchmark of the quantized-decode hot path on one MI355X.

Metric: achieved HBM GB/s of the INT4 matvec and the INT8-KV
(TurboQuant) decode attention, as a fraction of the 8 TB/s HBM3E peak.

Workload of the headline number: the Qwen3-4B decode
FFN block at batch 1 -- fused gate+up 2560 -> 2 x 9728 with SiLU, then down
9728 -> 2560, INT4 group-128 weights from N(0, 0.02), AWQ scales U[0.5, 2],
fp16 activations N(0,1) with 1 % of channels x20.  A step is one such FFN block
through the public FFN-block op imh_encode_ffn_block_int4 (encode_ffn_block):
two kernel launches, the gate/up one also writing the down projection's
operand image.  The weights are replicated over >= 512 MB of distinct buffers and the steps
rotate through them, so the MI355X's 256 MB Infinity Cache cannot serve them.

Bytes are counted as in the reference's kernel_bandwidth_bench
(ironmill-bench/examples/kernel_bandwidth_bench.rs:351-370): codes + f16
scales + f16 zeros + AWQ + x + y.

The JSON line also carries
  roofline     -- the dominant kernel (fused gate+up matvec with SiLU):
                  max(K, 1000) launches recorded into a HIP graph, replayed
                  between two HIP events on its stream after a warmup graph of
                  max(W, 2000) launches, time / launches;
  cpu_baseline -- the C oracle's dequantize-then-compute FFN step on the host
                  cores (weights dequantized once outside the timing);
  details      -- batch 4/8 FFN kernels, the prefill INT4 GEMM (M = 512 / 2048,
                  TFLOP/s against the 2.5 PFLOP/s dense f16 MFMA peak) and
                  TurboQuant attention at 32k.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense f16/bf16 matrix peak
H, F = 2560, 9728
INT4_BYTES_PER_ELEM = 0.5 + 4.0 / 128.0  # codes + f16 scale + f16 zero per 128


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gate_up_bytes(b):
    return 2 * F * H * INT4_BYTES_PER_ELEM + 2 * H + 2 * H * b + 2 * F * b


def down_bytes(b):
    return F * H * INT4_BYTES_PER_ELEM + 2 * F + 2 * F * b + 2 * H * b


def tq_bytes(b, ctx, nkv=8, nh=32, d=128):
    return b * (nkv * ctx * (2 * d + 12) + 2 * nh * d * 2)


def fp16_kv_bytes(b, ctx, nkv=8, nh=32, d=128):
    return b * (nkv * ctx * 2 * d * 2 + 2 * nh * d * 2)


def make_weights(seed):
    from ironmill_amd import quant
    rng = np.random.default_rng(seed)
    awq_h = rng.uniform(0.5, 2.0, H).astype(np.float32)
    awq_f = rng.uniform(0.5, 2.0, F).astype(np.float32)
    wg = (rng.standard_normal((F, H)) * 0.02).astype(np.float16).astype(np.float32)
    wu = (rng.standard_normal((F, H)) * 0.02).astype(np.float16).astype(np.float32)
    wd = (rng.standard_normal((H, F)) * 0.02).astype(np.float16).astype(np.float32)
    return (quant.quantize_int4(wg, awq_scales=awq_h), quant.quantize_int4(wu, awq_scales=awq_h),
            quant.quantize_int4(wd, awq_scales=awq_f))


def make_x(b, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, k)).astype(np.float32)
    idx = rng.choice(k, k // 100, replace=False)
    x[:, idx] *= 20.0
    return x.astype(np.float16)


def time_loop(dev, stream, fn, steps, warmup):
    """GPU time of `steps` calls fn(0..steps-1), back to back.

    The calls are recorded into a HIP graph (imh_stream_begin/end_capture) and
    replayed, so the device runs them without host launch gaps; a warmup graph
    of `warmup` calls runs first.  HIP events on the same stream bracket the
    timed replay.  Returns total ms.
    """
    fn(0)  # any scratch memory an op needs exists before capture
    stream.sync()
    if warmup > 0:
        wg = stream.capture(lambda: [fn(i) for i in range(warmup)])
        wg.launch()
    g = stream.capture(lambda: [fn(i) for i in range(steps)])
    stream.sync()
    s, e = dev.event(), dev.event()
    s.record(stream)
    g.launch()
    e.record(stream)
    stream.sync()
    return s.elapsed_ms(e)


def eager_loop(dev, stream, fn, steps, warmup):
    """As time_loop but with host launches (rocprofv3 counter collection sees only
    non-graph dispatches).  Returns total ms."""
    for i in range(warmup):
        fn(i)
    stream.sync()
    s, e = dev.event(), dev.event()
    s.record(stream)
    for i in range(steps):
        fn(i)
    e.record(stream)
    stream.sync()
    return s.elapsed_ms(e)


def cpu_baseline(qg, qu, qd, seconds, single_seconds=4.0):
    """The reference's CPU path (dequantize to f16 once, then f32 matvecs) on the host cores:
    a bounded multi-threaded sample, then a single-thread one."""
    import oracle as O
    cores = os.cpu_count() or 1
    threads = min(cores, 16)   # the GPU box's CPU share is 16 threads
    wg = O.dequant_affine_int4(qg.data, qg.scales_f32, qg.zeros_f32, F, H)
    wu = O.dequant_affine_int4(qu.data, qu.scales_f32, qu.zeros_f32, F, H)
    wd = O.dequant_affine_int4(qd.data, qd.scales_f32, qd.zeros_f32, H, F)
    x = make_x(1, H, 7)

    def run(nthreads, budget):
        reps, t0 = 0, time.perf_counter()
        while True:
            g = O.matvec_f16w(wg, x, qg.awq, nthreads=nthreads)
            u = O.matvec_f16w(wu, x, qg.awq, nthreads=nthreads)
            act = (g / (1.0 + np.exp(-g)) * u).astype(np.float16)
            O.matvec_f16w(wd, act, qd.awq, nthreads=nthreads)
            reps += 1
            if time.perf_counter() - t0 >= budget:
                return reps, (time.perf_counter() - t0) / reps

    reps, dt = run(threads, seconds)
    reps1, dt1 = run(1, single_seconds)
    nbytes = gate_up_bytes(1) + down_bytes(1)
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s (INT4 bytes model, FFN step batch 1)",
            "cores": cores, "threads": threads, "kind": "port",
            "single_thread": {"value": round(nbytes / dt1 / 1e9, 3), "ms_per_step": round(1e3 * dt1, 2),
                              "steps": reps1},
            "sample": f"{reps} Qwen3-4B FFN steps (gate+up+SiLU+down, batch 1) in {reps * dt:.1f} s on "
                      f"{threads} of {cores} host threads, {1e3 * dt:.1f} ms/step; C oracle, weights "
                      f"dequantized to f16 once outside the timing"}


def bench_attention(dev, stream, ops, batch, ctx, steps, warmup, layers, eager=False):
    """TurboQuant decode attention over `layers` distinct caches (rotated)."""
    nkv, nh, d = 8, 32, 128
    tq = ops.TurboQuantModel(dev, d, 8, 42)
    rng = np.random.default_rng(ctx + batch)
    caches = []
    chunk = 4096
    for _ in range(layers):
        c = ops.TurboQuantKvCache(dev, batch, nkv, d, ctx)
        for p0 in range(0, ctx, chunk):
            t = min(chunk, ctx - p0)
            kv = (rng.standard_normal((batch, t, nkv, d))).astype(np.float16)
            kd = dev.upload(kv)
            ops.encode_turboquant_cache_write(stream, tq, c, kd, t, p0, True)
            ops.encode_turboquant_cache_write(stream, tq, c, kd, t, p0, False)
            stream.sync()
        caches.append(c)
    q = dev.upload(rng.standard_normal((batch, nh, d)).astype(np.float16))
    out = dev.empty((batch, nh, d), np.float16)
    scale = 1.0 / math.sqrt(d)

    def step(i):
        ops.encode_turboquant_attention(stream, tq, caches[i % layers], q, nh, ctx, out, scale)

    total = (eager_loop if eager else time_loop)(dev, stream, step, steps, warmup)
    ms = total / steps
    gbs = tq_bytes(batch, ctx) / (ms * 1e-3) / 1e9
    return {"batch": batch, "ctx": ctx, "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": tq_bytes(batch, ctx), "launches": steps,
            "warmup_launches": warmup}


def bench_tq_prefill(dev, stream, ops, batch, ctx, tokens, steps, warmup, eager=False):
    """TurboQuant causal attention of a prefill chunk: the last `tokens` positions of a
    ctx-position cache attend to their prefixes (imh_encode_turboquant_attention_tokens)."""
    nkv, nh, d = 8, 32, 128
    tq = ops.TurboQuantModel(dev, d, 8, 42)
    rng = np.random.default_rng(ctx + tokens)
    c = ops.TurboQuantKvCache(dev, batch, nkv, d, ctx)
    for p0 in range(0, ctx, 4096):
        t = min(4096, ctx - p0)
        kd = dev.upload(rng.standard_normal((batch, t, nkv, d)).astype(np.float16))
        ops.encode_turboquant_cache_write(stream, tq, c, kd, t, p0, True)
        ops.encode_turboquant_cache_write(stream, tq, c, kd, t, p0, False)
        stream.sync()
    q = dev.upload(rng.standard_normal((batch, tokens, nh, d)).astype(np.float16))
    out = dev.empty((batch, tokens, nh, d), np.float16)

    def step(i):
        ops.encode_turboquant_attention(stream, tq, c, q, nh, ctx, out, 1.0 / math.sqrt(d), token_count=tokens)

    ms = (eager_loop if eager else time_loop)(dev, stream, step, steps, warmup) / steps
    # (query row, position) pairs attended: sum over tokens of their causal lengths
    pairs = batch * nh * sum(ctx - tokens + t + 1 for t in range(tokens))
    return {"batch": batch, "ctx": ctx, "tokens": tokens, "us": round(ms * 1e3, 2),
            "Gpairs/s": round(pairs / (ms * 1e-3) / 1e9, 2),
            "cache_passes_GB/s": round(tq_bytes(batch, ctx) / (ms * 1e-3) / 1e9, 1)}


def bench_fp16_attention(dev, stream, ops, batch, ctx, steps, warmup, layers, eager=False):
    """FP16-KV decode attention (fused_sdpa / FlashDecoding) over `layers` distinct caches."""
    nkv, nh, d = 8, 32, 128
    rng = np.random.default_rng(ctx + batch + 1)
    caches = []
    chunk = 4096
    for _ in range(layers):
        c = ops.Fp16KvCache(dev, batch, nkv, d, ctx)
        for p0 in range(0, ctx, chunk):
            t = min(chunk, ctx - p0)
            kd = dev.upload(rng.standard_normal((batch, t, nkv, d)).astype(np.float16))
            ops.encode_kv_scatter(stream, c, kd, t, p0, True)
            ops.encode_kv_scatter(stream, c, kd, t, p0, False)
            stream.sync()
        caches.append(c)
    q = dev.upload(rng.standard_normal((batch, nh, d)).astype(np.float16))
    out = dev.empty((batch, nh, d), np.float16)

    def step(i):
        ops.encode_fp16_attention(stream, caches[i % layers], q, nh, ctx, out, attn_scale=1.0 / math.sqrt(d))

    ms = (eager_loop if eager else time_loop)(dev, stream, step, steps, warmup) / steps
    nbytes = fp16_kv_bytes(batch, ctx)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"batch": batch, "ctx": ctx, "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes, "launches": steps, "warmup_launches": warmup}


GEMM_PEAK_TFS = {"f16": 2500.0, "bf16": 2500.0, "fp8": 5000.0}   # MI355X dense MFMA peaks


def bf16_bits(x32):
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x32, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bench_gemm(dev, stream, ops, m, kk, nn, prec, steps, warmup, eager=False, replicas=2):
    """Prefill INT4 GEMM: X [m, kk] N(0,1), W INT4 g128 [nn, kk] without AWQ, through
    imh_affine_gemm_int4 at `prec` (f16: x / y f16; bf16 and fp8: x / y bf16)."""
    rng = np.random.default_rng(31 * m + kk)
    Ws = [random_int4(dev, ops, rng, nn, kk, awq=False) for _ in range(replicas)]
    x32 = rng.standard_normal((m, kk)).astype(np.float32)
    xm = dev.upload(x32.astype(np.float16) if prec == "f16" else bf16_bits(x32))
    ym = dev.empty((m, nn), np.uint16)
    code = {"f16": ops.GEMM_F16, "bf16": ops.GEMM_BF16, "fp8": ops.GEMM_FP8_E4M3}[prec]

    def gm(i):
        ops.encode_affine_gemm_int4(stream, xm, m, Ws[i % replicas], ym, code)

    us = 1e3 * (eager_loop if eager else time_loop)(dev, stream, gm, steps, warmup) / steps
    tfs = 2.0 * m * nn * kk / (us * 1e-6) / 1e12
    return {"precision": prec, "us": round(us, 2), "TFLOP/s": round(tfs, 1),
            "frac": round(tfs / GEMM_PEAK_TFS[prec], 4), "peak_TFLOP/s": GEMM_PEAK_TFS[prec]}


def bench_valu_ab(dev, stream, ops, steps, warmup, eager=False, only=None):
    """Design A/B of the decode matvec: the library's MFMA kernels (imh_encode_affine_projection_int4)
    against the VALU-dot wavefront-reduction matvec (imh_diag_valu_matvec) on the same weights
    (rotating over >= 512 MB), Qwen3-4B gate (2560 -> 9728) at batch 1, 4 and 8 and O
    (4096 -> 2560) at batch 1; the two outputs' rel-L2 distance as a check."""
    out = {}
    rng = np.random.default_rng(77)
    for n, k, batches in ((F, H, (1, 4, 8)), (H, 4096, (1,))):
        nbytes = n * k // 2
        reps = max(2, math.ceil(512e6 / nbytes))
        Ws = [random_int4(dev, ops, rng, n, k) for _ in range(reps)]
        for b in batches:
            if only and (n, k, b) != only:
                continue
            x = dev.upload(make_x(b, k, 5 + b))
            ys = [dev.empty((b, n), np.float16) for _ in range(2)]
            for name, fn in (("mfma", ops.encode_projection), ("valu", ops.diag_valu_matvec)):
                y = ys[0 if name == "mfma" else 1]
                us = 1e3 * (eager_loop if eager else time_loop)(
                    dev, stream, lambda i, fn=fn, y=y: fn(stream, x, Ws[i % reps], y, b), steps, warmup) / steps
                gbs = (nbytes + n * (k // 128) * 4 + 2 * b * (k + n) + 2 * k) / (us * 1e-6) / 1e9
                out[f"{name}_n{n}_k{k}_b{b}"] = {"us": round(us, 2), "GB/s": round(gbs, 1),
                                                 "frac": round(gbs / HBM_PEAK_GBS, 4)}
            stream.sync()
            a, v = ys[0].read().astype(np.float64), ys[1].read().astype(np.float64)
            out[f"rel_l2_n{n}_k{k}_b{b}"] = float(np.linalg.norm(a - v) / max(np.linalg.norm(a), 1e-30))
    return out


def bench_probe(dev, stream, ops, steps, warmup, sweep=True):
    """Streaming probe (imh_diag_stream_read): the batch-1 gate+up and down weight bytes read
    with no compute, rotating over >= 512 MB of buffers like the matvec measurement.  `kernel`:
    the row-band matvec's own launch (one band of rows per CU; gate+up: 4 waves per weight,
    down: 8).  With `sweep`: TILE
    shapes of 8 / 16 rows, 1-4 tiles per workgroup and 1-16 waves, and FLAT grids of contiguous
    runs (the best of each reported as *_best)."""
    sink = dev.empty((1,), np.uint32)
    out = {}
    # per-launch floor: 256 workgroups reading 4 KiB in all
    tiny = dev.empty((4096,), np.uint8)
    us = 1e3 * time_loop(dev, stream, lambda i: ops.diag_stream_read(
        stream, tiny, 64, 128, sink, mode=ops.PROBE_FLAT, grid=256, threads=256), steps, warmup) / steps
    out["launch_floor"] = {"us": round(us, 2), "bytes": 4096, "grid": 256, "threads": 256}
    cus = dev.info()["compute_units"]
    cases = [("gate_up", F, H, 2, 4), ("down", H, F, 1, 8)]
    for name, n, k, nmat, own in cases:
        nbytes = nmat * n * k // 2
        reps = max(2, math.ceil(512e6 / nbytes))
        bufs = [dev.empty((nbytes,), np.uint8) for _ in range(reps)]
        G = k // 128
        runs = [("kernel", dict(mode=ops.PROBE_BAND, nmat=nmat, waves=own, grid=cus))]
        if sweep:
            for rows in (16, 8):
                for tiles in (1, 2, 4):
                    for waves in (1, 2, 4, 8, 16):
                        units = tiles * (G if rows == 16 else G // 2)
                        if waves * nmat > 16 or -(-units // waves) > 32 or -(-units // waves) < 2:
                            continue
                        runs.append((f"tile_r{rows}_t{tiles}_w{waves}",
                                     dict(mode=ops.PROBE_TILE, nmat=nmat, rows=rows, tiles=tiles, waves=waves)))
            runs += [(f"flat_g{g}_t{t}", dict(mode=ops.PROBE_FLAT, grid=g, threads=t))
                     for t in (256, 512, 1024) for g in (256, 512, 1024, 2048)]
        best = {}
        for label, shp in runs:
            def fn(i, shp=shp):
                ops.diag_stream_read(stream, bufs[i % reps], nmat * n if shp["mode"] == ops.PROBE_FLAT else n, k,
                                     sink, **shp)

            us = 1e3 * time_loop(dev, stream, fn, steps, warmup) / steps
            gbs = nbytes / (us * 1e-6) / 1e9
            key = f"{name}_{label}"
            out[key] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "bytes": nbytes, **{k_: v for k_, v in shp.items() if k_ != "mode"}}
            kind = label.split("_")[0]
            if kind != "kernel" and (kind not in best or us < out[best[kind]]["us"]):
                best[kind] = key
        for kind, key in best.items():
            out[f"{name}_{kind}_best"] = dict(out[key], case=key)
        del bufs
    return out


# Qwen3-4B shape of the decode-step measurement (cfg 5)
Q3 = dict(hidden_size=2560, intermediate_size=9728, num_layers=36, num_heads=32, num_kv_heads=8, head_dim=128,
          vocab_size=151936, rms_eps=1e-6, rope_theta=1e6)


def decode_step_bytes(b, ctx, cfg=Q3):
    """HBM bytes of one decode step: every INT4 weight (codes + f16 scale/zero per 128) and the
    whole TurboQuant cache each sequence attends over (268 B per position and kv head)."""
    H, F, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_layers"]
    qd, kvd = cfg["num_heads"] * cfg["head_dim"], cfg["num_kv_heads"] * cfg["head_dim"]
    per_layer = qd * H + 2 * kvd * H + H * qd + 2 * F * H + H * F
    weights = (L * per_layer + cfg["vocab_size"] * H) * INT4_BYTES_PER_ELEM
    kv = b * L * cfg["num_kv_heads"] * ctx * (2 * cfg["head_dim"] + 12)
    return weights + kv


def random_int4(dev, ops, rng, n, k, awq=True):
    """Synthetic INT4 weight in the upload layout: random codes, f16 scales in [1e-3, 3e-3],
    integer zero-points 0..15, AWQ scales in [0.5, 2] (awq True: new ones; a device buffer: that
    one, shared with another weight of the same input; False: none)."""
    data = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    sc = rng.uniform(1e-3, 3e-3, (n, k // 128)).astype(np.float16)
    zp = rng.integers(0, 16, size=(n, k // 128)).astype(np.float16)
    if awq is True:
        a = dev.upload(rng.uniform(0.5, 2.0, k).astype(np.float16))
    else:
        a = None if awq is False else awq
    return ops.AffineQuantizedWeight.from_pointers(dev.upload(data), dev.upload(sc), dev.upload(zp), a, n, k)


def bench_decode(dev, stream, ops, batch, ctx, steps, warmup, kv_cache="turboquant", graph=True):
    """Decode step of a Qwen3-4B-shaped model (36 layers, random INT4 weights incl. the LM head,
    QK-norm, TurboQuant KV cache filled to `ctx` positions): one step captured as a HIP graph and
    replayed once per token, timed with HIP events over `steps` replays."""
    cfg = dict(Q3, batch=batch, max_seq_len=ctx + steps + warmup + 8)
    rng = np.random.default_rng(2024)
    H, F, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_layers"]
    qd, kvd, hd = cfg["num_heads"] * cfg["head_dim"], cfg["num_kv_heads"] * cfg["head_dim"], cfg["head_dim"]
    d = ops.Decoder(dev, kv_cache=kv_cache, **cfg)
    keep = []

    def norm(n):
        return dev.upload(rng.uniform(0.8, 1.2, n).astype(np.float16))

    for l in range(L):
        # Q/K/V and gate/up read one activation each, so each set shares its AWQ scales
        q = random_int4(dev, ops, rng, qd, H)
        g = random_int4(dev, ops, rng, F, H)
        w = dict(input_norm=norm(H), post_attn_norm=norm(H), q_norm=norm(hd), k_norm=norm(hd),
                 q_proj=q, k_proj=random_int4(dev, ops, rng, kvd, H, awq=q.awq_scales),
                 v_proj=random_int4(dev, ops, rng, kvd, H, awq=q.awq_scales),
                 o_proj=random_int4(dev, ops, rng, H, qd, awq=False),
                 gate_proj=g, up_proj=random_int4(dev, ops, rng, F, H, awq=g.awq_scales),
                 down_proj=random_int4(dev, ops, rng, H, F))
        d.set_layer(l, **w)
        keep.append(w)
    emb = dev.upload((rng.standard_normal((cfg["vocab_size"], H)) * 0.05).astype(np.float16))
    lm = random_int4(dev, ops, rng, cfg["vocab_size"], H, awq=False)
    d.set_model(emb, norm(H), lm)
    # the cache of every layer filled to ctx positions from random K/V projections
    kv = dev.upload(rng.standard_normal((batch, ctx, cfg["num_kv_heads"], hd)).astype(np.float16))
    kv2 = dev.upload(rng.standard_normal((batch, ctx, cfg["num_kv_heads"], hd)).astype(np.float16))
    for l in range(L):
        d.write_kv(stream, l, kv, kv2, ctx, 0)
    stream.sync()
    del kv, kv2
    tok = dev.upload(rng.integers(0, cfg["vocab_size"], batch).astype(np.uint32))
    logits = dev.empty((batch, cfg["vocab_size"]), np.float16)
    start = np.full(batch, ctx, np.int32)
    d.reset(stream, start)
    d.step(stream, tok, logits)           # sizes the stream's scratch memory
    stream.sync()
    d.reset(stream, start)
    s, e = dev.event(), dev.event()
    ms = float("nan")
    if graph:
        g = stream.capture(lambda: d.step(stream, tok, logits))
        for _ in range(warmup):
            g.launch(stream)
        stream.sync()
        s.record(stream)
        for _ in range(steps):
            g.launch(stream)
        e.record(stream)
        stream.sync()
        ms = s.elapsed_ms(e) / steps
    # eager encode of the same step (host launches, no graph), for the launch-overhead picture
    d.reset(stream, start)
    s.record(stream)
    for _ in range(5):
        d.step(stream, tok, logits)
    e.record(stream)
    stream.sync()
    ms_eager = s.elapsed_ms(e) / 5
    nbytes = decode_step_bytes(batch, ctx)
    out = {"batch": batch, "ctx": ctx, "kv_cache": kv_cache, "ms_per_step": round(ms, 4),
           "tok_per_s": round(batch / (ms * 1e-3), 1), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
           "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": int(nbytes),
           "ms_per_step_eager": round(ms_eager, 4)}
    d.close()
    del keep
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-details", action="store_true")
    ap.add_argument("--replicas", type=int, default=0,
                    help="weight copies rotated through (default: enough for >= 512 MB, beyond the "
                         "256 MB Infinity Cache; 1 measures a cache-resident matrix)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the Qwen3-4B decode-step lines (B=1 and 8, ctx 8k), for profiling")
    ap.add_argument("--attention-only", choices=["tq", "fp16", "tq_prefill"],
                    help="only the decode attention at ctx 32k and --batch (tq_prefill: the causal attention of a 512- or 64-token chunk at ctx 2k / 8k)")
    ap.add_argument("--eager", action="store_true",
                    help="with --attention-only / --kernel: host launches instead of a graph (counter runs)")
    ap.add_argument("--decode-batches", type=int, nargs="+", default=[1, 8])
    ap.add_argument("--decode-eager", action="store_true",
                    help="with --decode-only: time 5 eager steps only (no graph capture; for kernel traces)")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the prepared fused gate+up kernel loop (same as --kernel gate_up)")
    ap.add_argument("--proj", type=int, nargs=2, metavar=("N", "K"),
                    help="with --kernel proj: the INT4 projection of an N x K weight (no AWQ; LM head: 151936 2560)")
    ap.add_argument("--kernel", choices=["gate_up", "down", "int8", "q8", "gemm", "probe", "valu_ab", "proj"],
                    help="one kernel alone, for rocprofv3 runs: the batch-B fused gate+up or down "
                         "matvec, the INT8 down-shape matvec, the INT4 x Q8 gate-shape "
                         "quantize + matvec, the prefill GEMM (--gemm-*), the streaming probe, or the MFMA / "
                         "VALU-dot matvec A/B; with --eager the launches are host launches (counter "
                         "runs see only those)")
    ap.add_argument("--ab-case", type=int, nargs=3, metavar=("N", "K", "B"),
                    help="with --kernel valu_ab: only this shape (counter runs)")
    ap.add_argument("--gemm-m", type=int, default=2048)
    ap.add_argument("--gemm-shape", choices=["gate", "down"], default="gate",
                    help="K=2560 N=9728 (gate) or K=9728 N=2560 (down)")
    ap.add_argument("--gemm-precision", choices=["f16", "bf16", "fp8"], default="bf16")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only 5 device-to-device copies of 256 MiB (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against a known byte count), then exit")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch
        a = torch.ones(64 << 20, dtype=torch.int32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copy calibration: 5 copies of {a.numel() * 4} bytes")
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the hot path has no multi-GPU code: each GPU would hold its own column shard of "
              "every projection and its own heads of the KV cache)",
              file=sys.stderr)
        sys.exit(2)

    from ironmill_amd import Device, ops
    dev = Device(0)
    stream = dev.stream()
    info = dev.info()
    log(f"device {info['arch']} CUs={info['compute_units']}")

    if args.attention_only == "tq_prefill":
        for ctx, tokens in ((2048, 512), (8192, 512), (8192, 64)):
            r = bench_tq_prefill(dev, stream, ops, args.batch, ctx, tokens, max(5, args.steps // 10), 3,
                                 eager=args.eager)
            log(f"tq prefill attention B={args.batch} ctx={ctx} T={tokens}: {r['us']} us")
            print(json.dumps({f"tq_prefill_attention_b{args.batch}_ctx{ctx}_t{tokens}": r}), flush=True)
        return
    if args.attention_only:
        fn = bench_attention if args.attention_only == "tq" else bench_fp16_attention
        layers = max(1, min(8, 16 // args.batch))
        r = fn(dev, stream, ops, args.batch, 32768, args.steps, args.warmup, layers, eager=args.eager)
        log(f"{args.attention_only} attention B={args.batch} ctx=32k: {r['us']} us {r['GB/s']} GB/s")
        print(json.dumps({f"{args.attention_only}_attention_b{args.batch}_ctx32k": r}), flush=True)
        return
    if args.decode_only:
        for bb in args.decode_batches:
            r = bench_decode(dev, stream, ops, bb, 8192, max(20, args.steps // 10), 3, graph=not args.decode_eager)
            log(f"decode step B={bb} ctx=8k: {r['ms_per_step']} ms ({r['tok_per_s']} tok/s, "
                f"{r['GB/s']} GB/s); eager encode {r['ms_per_step_eager']} ms")
            print(json.dumps({f"decode_step_b{bb}_ctx8k": r}), flush=True)
        return

    if args.kernel_only:
        args.kernel = "gate_up"
    if args.kernel == "gemm":
        kk, nn = (H, F) if args.gemm_shape == "gate" else (F, H)
        r = bench_gemm(dev, stream, ops, args.gemm_m, kk, nn, args.gemm_precision, args.steps, args.warmup,
                       eager=args.eager)
        log(f"GEMM {args.gemm_precision} M={args.gemm_m} K={kk} N={nn}: {r['us']} us {r['TFLOP/s']} TFLOP/s")
        print(json.dumps({f"gemm_{args.gemm_precision}_m{args.gemm_m}_k{kk}_n{nn}": r}), flush=True)
        return
    if args.kernel == "valu_ab":
        only = tuple(args.ab_case) if args.ab_case else None
        r = bench_valu_ab(dev, stream, ops, args.steps, args.warmup, eager=args.eager, only=only)
        for k_, v in r.items():
            log(f"{k_}: {v}")
        print(json.dumps({"matvec_mfma_vs_valu": r}), flush=True)
        return
    if args.kernel == "probe":
        r = bench_probe(dev, stream, ops, args.steps, args.warmup)
        for k_, v in r.items():
            log(f"probe {k_}: {v['us']} us {v.get('GB/s', '-')} GB/s")
        print(json.dumps({"stream_probe": r}), flush=True)
        return

    if args.kernel == "proj":
        # one INT4 projection (e.g. the LM head) at --batch, random codes and f16 scales / zero
        # points in the upload layout, rotating over >= 512 MB of weights
        B = args.batch
        nn, kk = args.proj or (151936, 2560)
        rng = np.random.default_rng(7)
        per = nn * kk * INT4_BYTES_PER_ELEM
        Wp = [random_int4(dev, ops, rng, nn, kk, awq=False) for _ in range(max(2, math.ceil(512e6 / per)))]
        xp = dev.upload(make_x(B, kk, 95))
        yp = dev.empty((B, nn), np.float16)
        tot = (eager_loop if args.eager else time_loop)(
            dev, stream, lambda i: ops.encode_projection(stream, xp, Wp[i % len(Wp)], yp, B), args.steps, args.warmup)
        us = 1e3 * tot / args.steps
        nb = per + 2 * B * (kk + nn)
        gbs = nb / (us * 1e-6) / 1e9
        log(f"INT4 projection {nn}x{kk} B={B}: {us:.2f} us  {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f} %)")
        print(json.dumps({"kernel": f"INT4 projection {nn}x{kk}", "batch": B, "us": round(us, 3),
                          "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": int(nb),
                          "launches": args.steps, "eager": args.eager}))
        return

    if args.kernel == "int8":
        # INT8 sensitive-layer weights at the down shape (K 9728 -> N 2560), weights rotating
        # over replicas of 512 MB in total
        from ironmill_amd import quant as Q
        B = args.batch
        q8w = Q.quantize_int8((np.random.default_rng(8).standard_normal((H, F)) * 0.02).astype(np.float32))
        W8 = [ops.AffineInt8Weight(dev, q8w) for _ in range(max(2, math.ceil(512e6 / q8w.data.nbytes)))]
        a8 = dev.upload(make_x(B, F, 97))
        y8 = dev.empty((B, H), np.float16)
        tot = (eager_loop if args.eager else time_loop)(
            dev, stream, lambda i: ops.encode_projection_int8(stream, a8, W8[i % len(W8)], y8, B), args.steps,
            args.warmup)
        us = 1e3 * tot / args.steps
        nb = q8w.data.nbytes + q8w.scales.nbytes * 2 + B * 2 * (F + H)
        gbs = nb / (us * 1e-6) / 1e9
        log(f"INT8 down kernel B={B}: {us:.2f} us  {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f} %)")
        print(json.dumps({"kernel": "int8w_band_kernel" if B <= 3 else "int8w_matvec_kernel", "batch": B,
                          "us": round(us, 3), "GB/s": round(gbs, 1), "bytes": nb, "launches": args.steps,
                          "eager": args.eager}))
        return

    if args.kernel == "q8":
        # INT4 x Q8 at the gate shape (K 2560 -> N 9728): the quantize launch and the matvec
        from ironmill_amd import quant as Q
        B = args.batch
        qg0 = Q.quantize_int4((np.random.default_rng(8).standard_normal((F, H)) * 0.02).astype(np.float32))
        W4 = [ops.AffineQuantizedWeight(dev, qg0) for _ in range(max(2, math.ceil(512e6 / qg0.data.nbytes)))]
        xq = dev.upload(make_x(B, H, 96))
        q8d, q8s = dev.empty((B, H), np.int8), dev.empty((B, H // 128), np.float32)
        gq = dev.empty((B, F), np.float16)

        def q8_step(i):   # the one-launch op: quantize while staging, then the integer matvec
            ops.encode_projection_int4_q8(stream, xq, W4[i % len(W4)], gq, B)

        tot = (eager_loop if args.eager else time_loop)(dev, stream, q8_step, args.steps, args.warmup)
        us = 1e3 * tot / args.steps
        nb = int(F * H * INT4_BYTES_PER_ELEM + B * 2 * (H + F))
        gbs = nb / (us * 1e-6) / 1e9
        log(f"INT4xQ8 gate B={B}: {us:.2f} us (1 launch)  {gbs:.0f} GB/s")
        print(json.dumps({"kernel": "int4xq8_band_kernel<FQ> (f16 rows quantized in the launch)", "batch": B,
                          "us": round(us, 3), "GB/s": round(gbs, 1), "bytes": nb, "launches": args.steps,
                          "eager": args.eager}))
        return

    B = args.batch
    qg, qu, qd = make_weights(1234)
    per_copy = (qg.data.nbytes + qg.scales.nbytes * 2) * 3
    reps = args.replicas or max(1, math.ceil(512e6 / per_copy))
    log(f"uploading {reps} weight replicas ({reps * per_copy / 1e6:.0f} MB)")
    W = [(ops.AffineQuantizedWeight(dev, qg), ops.AffineQuantizedWeight(dev, qu),
          ops.AffineQuantizedWeight(dev, qd)) for _ in range(reps)]
    x = dev.upload(make_x(B, H, 99))
    act = dev.empty((B, F), np.float16)
    y = dev.empty((B, H), np.float16)

    # ---- dominant kernel: fused gate+up matvec (one launch per op) ----
    def gate_up_kernel(i):
        g, u, _ = W[i % reps]
        ops.encode_fused_ffn_gate_up_act_int4(stream, x, g, u, act, B)

    if args.kernel == "down":
        a0 = dev.upload(make_x(B, F, 98))

        def down_only(i):
            ops.encode_projection(stream, a0, W[i % reps][2], y, B)

        tot = (eager_loop if args.eager else time_loop)(dev, stream, down_only, args.steps, args.warmup)
        us = 1e3 * tot / args.steps
        gbs = down_bytes(B) / (us * 1e-6) / 1e9
        log(f"down kernel B={B}: {us:.2f} us  {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f} %)")
        print(json.dumps({"kernel": ("int4_band_kernel" if B <= 2 else "int4_prep_plain + int4_splitk_kernel + combine"
                                     if B <= 8 else "int4_matvec_kernel") + " (down projection)",
                          "batch": B, "us": round(us, 3),
                          "GB/s": round(gbs, 1), "launches": args.steps, "eager": args.eager}))
        return

    # the roofline loop does not follow --steps: >= 1000 timed launches (~9 ms) after a warmup
    # graph of >= 2000 (~18 ms) -- the first tens of ms of back-to-back launches run at lower
    # clocks -- so the average is the sustained rate; the FFN step timed next starts settled
    ksteps = max(args.steps, 1000)
    kwarm = max(args.warmup, 2000)
    tot = (eager_loop if args.eager and args.kernel else time_loop)(dev, stream, gate_up_kernel, ksteps, kwarm)
    k_us = 1e3 * tot / ksteps
    k_bytes = gate_up_bytes(B)
    k_gbs = k_bytes / (k_us * 1e-6) / 1e9
    log(f"gate+up kernel: {k_us:.2f} us  {k_gbs:.0f} GB/s ({100 * k_gbs / HBM_PEAK_GBS:.1f} %)")
    if args.kernel == "gate_up":
        print(json.dumps({"kernel": ("int4_band_kernel" if B <= 8 else "int4_matvec_kernel") + "<2, SILU> (gate+up)",
                          "batch": B, "us": round(k_us, 3),
                          "GB/s": round(k_gbs, 1), "launches": ksteps, "eager": args.eager}))
        return

    # ---- the step: FFN block through the public ops ----
    def ffn_step(i):
        g, u, d = W[i % reps]
        ops.encode_ffn_block_int4(stream, x, g, u, d, act, y, B)

    total_ms = time_loop(dev, stream, ffn_step, args.steps, args.warmup)
    ms = total_ms / args.steps
    step_bytes = gate_up_bytes(B) + down_bytes(B)
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"FFN step: {ms * 1e3:.2f} us  {value:.0f} GB/s")

    traffic = None
    tpath = os.path.join(REPO, "profiles", "traffic_gate_up_b1.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    details = {}
    if not args.no_details:
        # down projection kernel alone, and the FFN kernels at batch 4 / 8
        def down_kernel(i):
            ops.encode_projection(stream, act, W[i % reps][2], y, B)

        t = time_loop(dev, stream, down_kernel, args.steps, args.warmup)
        d_us = 1e3 * t / args.steps
        details["down_kernel_b%d" % B] = {"us": round(d_us, 2),
                                          "GB/s": round(down_bytes(B) / (d_us * 1e-6) / 1e9, 1)}
        for bb in (4, 8):
            xb = dev.upload(make_x(bb, H, 5 + bb))
            ab = dev.empty((bb, F), np.float16)

            def gu(i, xb=xb, ab=ab, bb=bb):
                g, u, _ = W[i % reps]
                ops.encode_fused_ffn_gate_up_act_int4(stream, xb, g, u, ab, bb)

            t = time_loop(dev, stream, gu, args.steps, args.warmup)
            us = 1e3 * t / args.steps
            details[f"gate_up_kernel_b{bb}"] = {"us": round(us, 2),
                                                "GB/s": round(gate_up_bytes(bb) / (us * 1e-6) / 1e9, 1)}
            ops.encode_fused_ffn_gate_up_act_int4(stream, xb, W[0][0], W[0][1], ab, bb)
            yb = dev.empty((bb, H), np.float16)

            def dn(i, ab=ab, yb=yb, bb=bb):
                ops.encode_projection(stream, ab, W[i % reps][2], yb, bb)

            t = time_loop(dev, stream, dn, args.steps, args.warmup)
            us = 1e3 * t / args.steps
            details[f"down_kernel_b{bb}"] = {"us": round(us, 2),
                                             "GB/s": round(down_bytes(bb) / (us * 1e-6) / 1e9, 1)}
        # INT8 sensitive-layer weights (down shape) and the INT4 x Q8 decode variant (gate shape)
        from ironmill_amd import quant as Q
        rng8 = np.random.default_rng(8)
        q8w = Q.quantize_int8((rng8.standard_normal((H, F)) * 0.02).astype(np.float32))
        W8 = [ops.AffineInt8Weight(dev, q8w) for _ in range(max(2, math.ceil(512e6 / q8w.data.nbytes)))]
        a1 = dev.upload(make_x(1, F, 97))
        t = time_loop(dev, stream, lambda i: ops.encode_projection_int8(stream, a1, W8[i % len(W8)], y, 1),
                      args.steps, args.warmup)
        us = 1e3 * t / args.steps
        nb = q8w.data.nbytes + q8w.scales.nbytes * 2 + 2 * F + 2 * H
        details["int8_down_kernel_b1"] = {"us": round(us, 2), "GB/s": round(nb / (us * 1e-6) / 1e9, 1),
                                          "bytes": nb}
        del W8
        qg0 = Q.quantize_int4((rng8.standard_normal((F, H)) * 0.02).astype(np.float32))
        W4 = [ops.AffineQuantizedWeight(dev, qg0) for _ in range(reps)]
        q8d, q8s = dev.empty((1, H), np.int8), dev.empty((1, H // 128), np.float32)
        g1 = dev.empty((1, F), np.float16)

        def q8_step(i):   # one launch: the f16 row quantized while staged
            ops.encode_projection_int4_q8(stream, x, W4[i % reps], g1, 1)

        def q8_pair(i):   # the two launches: quantize, then the matvec on the codes
            ops.encode_quantize_input_q8(stream, x, 1, H, q8d, q8s)
            ops.encode_affine_matvec_int4xq8(stream, q8d, q8s, 1, W4[i % reps], g1)

        nb = F * H * INT4_BYTES_PER_ELEM + 2 * H + 2 * F
        for key, fn, nl in (("int4xq8_gate_b1", q8_step, 1), ("int4xq8_gate_b1_two_launches", q8_pair, 2)):
            t = time_loop(dev, stream, fn, args.steps, args.warmup)
            us = 1e3 * t / args.steps
            details[key] = {"us": round(us, 2), "GB/s": round(nb / (us * 1e-6) / 1e9, 1), "launches": nl,
                            "bytes": int(nb)}
        del W4
        log(f"INT8 down B=1: {details['int8_down_kernel_b1']['us']} us; INT4xQ8 gate B=1: "
            f"{details['int4xq8_gate_b1']['us']} us one launch, "
            f"{details['int4xq8_gate_b1_two_launches']['us']} us quantize + matvec")
        # prefill INT4 GEMM: M tokens, bf16 and fp8-e4m3 (and f16, the projection op)
        for mm in (512, 2048):
            for (kk, nn) in ((H, F), (F, H)):
                for prec in ("bf16", "fp8", "f16"):
                    r = bench_gemm(dev, stream, ops, mm, kk, nn, prec, max(20, args.steps // 4), 3)
                    details[f"gemm_{prec}_m{mm}_k{kk}_n{nn}"] = r
                    log(f"prefill GEMM {prec} M={mm} K={kk} N={nn}: {r['us']} us {r['TFLOP/s']} TFLOP/s "
                        f"({100 * r['frac']:.1f} % of dense {prec} MFMA)")
        # the LM head (151936 x 2560, 206.6 MB) at one row: the INT4 decode matvec at its largest
        # Qwen3-4B shape, where the launch floor is a small share of the launch
        rng_lm = np.random.default_rng(7)
        lm_per = 151936 * H * INT4_BYTES_PER_ELEM
        WL = [random_int4(dev, ops, rng_lm, 151936, H, awq=False) for _ in range(3)]
        xl = dev.upload(make_x(1, H, 95))
        yl = dev.empty((1, 151936), np.float16)
        t = time_loop(dev, stream, lambda i: ops.encode_projection(stream, xl, WL[i % 3], yl, 1),
                      max(200, args.steps), max(200, args.warmup))
        us = 1e3 * t / max(200, args.steps)
        nb = lm_per + 2 * (H + 151936)
        details["lm_head_b1"] = {"us": round(us, 2), "GB/s": round(nb / (us * 1e-6) / 1e9, 1),
                                 "frac": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "bytes": int(nb),
                                 "launches": max(200, args.steps)}
        log(f"LM head B=1: {us:.2f} us ({details['lm_head_b1']['frac'] * 100:.1f} % of 8 TB/s)")
        del WL
        details["stream_probe"] = bench_probe(dev, stream, ops, max(50, args.steps // 2), args.warmup, sweep=False)
        del W
        stream.sync()
        # sustained rates: a warmup graph long enough for the clocks to settle
        # (measured: the first ~50 ms of back-to-back launches after the weight
        # benchmarks run up to 10 % slower than the steady state)
        # (~25 us per call at batch 1: 2000 warmup launches are ~50 ms, and 500
        # timed ones ~12 ms; ~200 us at batch 16)
        att_runs = {1: (max(500, args.steps), max(2000, args.warmup)),
                    16: (max(20, args.steps // 4), max(200, args.warmup))}
        for bb, layers in ((1, 8), (16, 1)):
            r = bench_attention(dev, stream, ops, bb, 32768, *att_runs[bb], layers)
            details[f"tq_attention_b{bb}_ctx32k"] = r
            log(f"TQ attention B={bb} ctx=32k: {r['us']} us {r['GB/s']} GB/s")
        for bb, layers in ((1, 8), (16, 1)):
            r = bench_fp16_attention(dev, stream, ops, bb, 32768, *att_runs[bb], layers)
            details[f"fp16_attention_b{bb}_ctx32k"] = r
            log(f"FP16-KV attention B={bb} ctx=32k: {r['us']} us {r['GB/s']} GB/s")
        for bb in (1, 8):
            r = bench_decode(dev, stream, ops, bb, 8192, max(20, args.steps // 10), 3)
            details[f"decode_step_b{bb}_ctx8k"] = r
            log(f"decode step B={bb} ctx=8k: {r['ms_per_step']} ms ({r['tok_per_s']} tok/s, "
                f"{r['GB/s']} GB/s)")
        log(json.dumps(details))

    cpu = None
    if not args.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline(qg, qu, qd, args.cpu_seconds)

    line = {
        "metric": "INT4 matvec & INT8-KV decode attn: achieved HBM GB/s (% peak); decode tok/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "qwen3-4b decode FFN block, INT4 g128 + AWQ (BASELINE configs[1])",
                   "batch": B, "gate_up": [H, 2, F], "down": [F, H], "group_size": 128,
                   "awq": True, "weight_replicas": reps},
        "roofline": {"bound": "hbm", "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": ("int4_band_kernel" if B <= 8 else "int4_matvec_kernel") + " (fused gate+up, SiLU, AWQ)",
                     "bytes_per_launch": k_bytes, "us_per_launch": round(k_us, 3), "launches": ksteps,
                     "warmup_launches": kwarm},
        "cpu_baseline": cpu,
        "details": details,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
