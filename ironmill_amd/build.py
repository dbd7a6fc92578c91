"""Build recipe for libironmill_hip.so (hipcc, gfx950).

Compiles every source under ironmill_amd/csrc into one shared library at
ironmill_amd/lib/libironmill_hip.so.  Runs on a machine without a GPU: hipcc
cross-compiles for gfx950.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libironmill_hip.so")
OBJDIR = os.path.join(HERE, "_build")

SOURCES = ["runtime.hip", "int4_matvec.hip", "int4_matvec_raw.hip", "int4_matvec_mt2.hip", "int4_matvec_band.hip", "int4_matvec_da.hip",
           "int4_gemm.hip",
           "int4_gemm_mx.hip", "int8_matvec.hip",
           "tq_kernels.hip", "fp16_attention.hip", "glue_kernels.hip", "decoder.hip",
           "tq_tables.cpp", "diag_probe.hip", "diag_valu_matvec.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -packed-fp32-ops: hipcc must not emit packed f32 VALU ops (they have given
# silent wrong results on these machines); the host pass ignores the feature.
# -amdgpu-kernarg-preload-count: the dispatcher places a kernel's leading
# scalar arguments (up to 14 SGPRs) in registers before its first
# instruction, so the loads that need them issue without waiting for the
# argument memory (~0.25 us per latency-bound launch; the code object keeps
# a 256-byte entry that loads them itself for dispatchers without preload).
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


# per-source additions: the attention kernels keep MFMA accumulators in VGPRs
# (the softmax rescale touches them every chunk; AGPR copies would cost 64 VALU)
EXTRA_FLAGS = {
    "tq_kernels.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def build(verbose: bool = False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
        lang = ["-x", "hip"]
        cmd = [HIPCC, *FLAGS, *EXTRA_FLAGS.get(src, []), *lang, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(obj)
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        # the host pass always warns about the gfx-only target feature
        lines = [l for l in text.splitlines() if "packed-fp32-ops" not in l]
        if lines and (verbose or p.returncode):
            print("\n".join(lines), file=sys.stderr)
        if p.returncode:
            failed.append(src)
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(failed))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
