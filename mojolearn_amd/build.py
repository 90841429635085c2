"""Build libmlgemm.so in place with hipcc for gfx950 (no GPU needed to compile).

Each translation unit is compiled to an object in a temporary directory, the units in
parallel (the skinny-M kernels instantiate many template variants and dominate the time),
then linked into mojolearn_amd/libmlgemm.so.
"""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libmlgemm.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # packed fp32 (v_pk_fma_f32 and friends) stays off in every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
SOURCES = ["gemv_nn.hip", "gemv_nt.hip", "gemv_mfma.hip", "gemv_packed.hip", "gemm_mfma.hip", "gemm_q8.hip", "kernels.hip", "follow.hip", "transport.hip", "stream_read.hip", "capi.hip"]


def _clean(stderr):
    return "\n".join(l for l in stderr.splitlines() if "packed-fp32-ops" not in l)


def build(verbose=False, extra=(), jobs=None):
    with tempfile.TemporaryDirectory(prefix="mlgemm_build_") as tmp:
        objs = [os.path.join(tmp, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        cmds = [[HIPCC, *FLAGS, *extra, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
        if verbose:
            for c in cmds:
                print(" ".join(c), flush=True)
        with ThreadPoolExecutor(max_workers=jobs or len(cmds)) as pool:
            results = list(pool.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds))
        for c, r in zip(cmds, results):
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed on {c[-3]}:\n" + _clean(r.stderr))
            if verbose and _clean(r.stderr).strip():
                print(_clean(r.stderr), file=sys.stderr)
        link = [HIPCC, "--offload-arch=gfx950", "-fPIC", "-shared", *objs, "-o", LIB + ".tmp"]
        if verbose:
            print(" ".join(link), flush=True)
        r = subprocess.run(link, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("hipcc link failed:\n" + _clean(r.stderr))
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
