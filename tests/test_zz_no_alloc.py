"""The allocation-free TurboQuant attention entry point against the ordinary one.

imh_encode_turboquant_attention_noalloc keeps its split partials in a fixed
per-GPU device array instead of the stream's scratch.  It runs the same
kernels with the same split count, so its output must equal
imh_encode_turboquant_attention's bit for bit.  Two calls in a row, the second
on a smaller input, check that the array's leftover contents (the first call's
partials) do not leak into the second.  Both calls go
through the C ABI (ctypes), as a binding would make them.
"""
import ctypes as C
import math

import numpy as np
import pytest

from ironmill_amd import _lib, ops
from ironmill_amd._lib import lib

pytestmark = pytest.mark.gpu

D = 128


def _cache(dev, stream, tq, batch, nkv, max_seq, ctx, seed):
    rng = np.random.default_rng(seed)
    cache = ops.TurboQuantKvCache(dev, batch, nkv, D, max_seq)
    cache.zero(stream)
    k = rng.standard_normal((batch, ctx, nkv, D)).astype(np.float16)
    v = rng.standard_normal((batch, ctx, nkv, D)).astype(np.float16)
    ops.encode_turboquant_cache_write_kv(stream, tq, cache, dev.upload(k), dev.upload(v), ctx, 0)
    stream.sync()
    return cache


def _call(fn, stream, tq, cache, qd, nh, seq_len, out, num_splits):
    rc = fn(stream.handle, tq.handle, C.byref(cache.c), C.c_void_p(qd.ptr), nh, seq_len, None,
            C.c_float(1.0 / math.sqrt(D)), C.c_void_p(out.ptr), num_splits)
    return rc


@pytest.mark.parametrize("num_splits", [0, 5])
def test_noalloc_matches_allocating_entry(dev, stream, num_splits):
    tq = ops.TurboQuantModel(dev, D, 8, 42)
    nkv, nh = 8, 32
    # first call: batch 4 at 4096 positions; second: batch 2 at 1000 (smaller)
    for batch, ctx, seed in ((4, 4096, 11), (2, 1000, 12)):
        print(f"noalloc case batch={batch} ctx={ctx} num_splits={num_splits}", flush=True)
        cache = _cache(dev, stream, tq, batch, nkv, ctx, ctx, seed)
        q = np.random.default_rng(seed + 100).standard_normal((batch, nh, D)).astype(np.float16)
        qd = dev.upload(q)
        ref = dev.empty(q.shape, np.float16)
        got = dev.empty(q.shape, np.float16)
        assert _call(lib.imh_encode_turboquant_attention, stream, tq, cache, qd, nh, ctx, ref, num_splits) == 0, \
            _lib.last_error()
        assert _call(lib.imh_encode_turboquant_attention_noalloc, stream, tq, cache, qd, nh, ctx, got,
                     num_splits) == 0, _lib.last_error()
        stream.sync()
        r, g = ref.read(), got.read()
        assert np.all(np.isfinite(g))
        assert np.array_equal(g.view(np.uint16), r.view(np.uint16)), \
            f"batch {batch} ctx {ctx}: {np.count_nonzero(g != r)} outputs differ"


def test_noalloc_rejects_oversized_shape(dev, stream):
    """More partials than the fixed array holds: IMH_EINVAL before any launch."""
    tq = ops.TurboQuantModel(dev, D, 8, 42)
    batch, nkv, nh, ctx = 64, 8, 32, 8192
    cache = ops.TurboQuantKvCache(dev, batch, nkv, D, ctx)   # contents unused: the call is refused
    q = dev.empty((batch, nh, D), np.float16)
    out = dev.empty((batch, nh, D), np.float16)
    # 64 x 32 heads x 32 splits x 520 B = 34 MB of partials > 4 MiB
    rc = _call(lib.imh_encode_turboquant_attention_noalloc, stream, tq, cache, q, nh, ctx, out, 32)
    assert rc == _lib.IMH_EINVAL
    assert "fixed scratch" in _lib.last_error()
