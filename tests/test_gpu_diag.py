"""The measurement aids of include/ironmill_diag.h on the GPU.

* imh_diag_valu_matvec (the VALU-dot design the MFMA kernels are measured
  against) computes the same projection: within the north star's rel-L2 1e-3
  of the oracle's CPU path and of the GPU weight layout's exact value, at the
  Qwen3-4B shapes it is timed on, with and without AWQ.
* imh_diag_stream_read runs in each launch shape it offers (no values to
  check: it only reads).
"""
import numpy as np
import pytest

import oracle as O
from conftest import assert_close
from ironmill_amd import IronmillError, ops, quant
from test_gpu_int4 import gpu_layout_y, make_weight, make_x, oracle_dense, upload_weight

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k,batch,awq", [
    (9728, 2560, 1, True),
    (9728, 2560, 4, False),
    (9728, 2560, 8, True),
    (2560, 4096, 1, True),
    (2560, 4096, 2, False),
    (1003, 2560, 3, True),   # bands that end in a partial 4-row slot
])
def test_valu_matvec_matches_oracle(dev, stream, n, k, batch, awq):
    print(f"valu matvec n={n} k={k} batch={batch} awq={awq}", flush=True)
    w, s = make_weight(n, k, seed=41 + batch, awq=awq)
    x16 = make_x(batch, k, seed=42)
    wt = upload_weight(dev, w, s)
    xd = dev.upload(x16)
    y = dev.empty((batch, n), np.float16)
    ops.diag_valu_matvec(stream, xd, wt, y, batch)
    stream.sync()
    got = y.read()
    wdq, awq16 = oracle_dense(w, s)
    assert_close(got, O.matvec_f16w(wdq, x16, awq16, nthreads=8), what="valu matvec vs CPU path", ulps=2)
    q = quant.quantize_int4(w, awq_scales=s)
    assert_close(got, gpu_layout_y(q, x16, awq16), what="valu matvec vs GPU layout")


def test_valu_matvec_refuses_unbuilt_shapes(dev, stream):
    w, _ = make_weight(64, 1024, seed=3)
    wt = upload_weight(dev, w, None)
    x = dev.upload(make_x(1, 1024, seed=4))
    y = dev.empty((1, 64), np.float16)
    with pytest.raises(IronmillError, match="k of 2560 or 4096"):
        ops.diag_valu_matvec(stream, x, wt, y, 1)


@pytest.mark.parametrize("mode,kw", [
    (ops.PROBE_TILE, dict(rows=16, tiles=1, waves=4)),
    (ops.PROBE_TILE, dict(rows=8, tiles=2, waves=2, nmat=2)),
    (ops.PROBE_FLAT, dict(grid=512, threads=256)),
    (ops.PROBE_BAND, dict(grid=256, waves=4, nmat=2)),
])
def test_stream_probe_runs(dev, stream, mode, kw):
    n, k = 2048, 2560
    nmat = kw.get("nmat", 1)
    src = dev.upload(np.random.default_rng(5).integers(0, 256, nmat * n * k // 2, dtype=np.uint8))
    sink = dev.upload(np.zeros(1, np.uint32))
    ops.diag_stream_read(stream, src, n, k, sink, mode=mode, **kw)
    stream.sync()
