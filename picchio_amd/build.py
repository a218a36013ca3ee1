"""Builds libpicchio_hip.so for gfx950 in-tree (hipcc, no JIT cache).

    python -m picchio_amd.build        # or picchio_amd.build.build()
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libpicchio_hip.so")
OBJ = os.path.join(HERE, "_build")
SOURCES = ["pk_i4.hip", "pk_moe.hip", "pk_dense.hip", "pk_engine.hip", "pk_decode.hip",
           "pk_prefill.hip", "pk_mfma.hip", "pk_sample.hip", "pk_exact.hip", "pk_container.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=off: every fused multiply-add in the kernels is an explicit
# fmaf, so results follow the reference's rounding, not the compiler's.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in the generated code.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-result", "-Wno-unused-command-line-argument"]


def _compile(src):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l and "unknown target feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msgs}")
    return obj, msgs


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        results = list(ex.map(_compile, SOURCES))
    for _, msgs in results:
        if verbose and msgs.strip():
            print(msgs)
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp,
           *[o for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, OUT)
    build_service()
    return OUT


SERVICE_SRC = os.path.join(HERE, "host", "picchio_service.c")
SERVICE_OUT = os.path.join(HERE, "picchio_service")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")


def build_service():
    """picchio's SERVICE=1 loop as a C program over the C-ABI (gcc, linked
    against the library next to it)."""
    tmp = SERVICE_OUT + ".tmp"
    cmd = [os.environ.get("CC", "gcc"), "-O2", "-std=c11", "-Wall", "-Wextra", "-I", INCLUDE, SERVICE_SRC,
           "-L", HERE, "-lpicchio_hip", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath-link,/opt/rocm/lib", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("service build failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, SERVICE_OUT)
    return SERVICE_OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
