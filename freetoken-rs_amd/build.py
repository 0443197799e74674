"""Build libfthip.so (the gfx950 HIP library behind include/ft_hip.h).

hipcc cross-compiles for gfx950 without a GPU. Objects go to
freetoken-rs_amd/_build/, the library to freetoken-rs_amd/lib/libfthip.so.

Flags:
  --offload-arch=gfx950          MI355X only (no other targets, no CUDA path)
  -ffp-contract=off              a*b+c stays two roundings unless fma() is
                                 written, so f32 expressions follow the Rust
                                 source they restate
  -target-feature -packed-fp32-ops  no v_pk_{add,mul,fma}_f32 generation
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib", "libfthip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["ft_runtime.cpp", "ft_gguf.cpp", "ft_hip_ops.hip", "ft_hip_fused.hip", "ft_hip_grouped.hip"]
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
             "-fno-fast-math", "-Wall", "-Wno-unused-function",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed: " + " ".join(cmd))
    # hipcc's host pass does not know the packed-fp32 feature and says so; keep
    # other warnings visible.
    msgs = [l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if msgs and verbose:
        print("\n".join(msgs))


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    objs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            continue
        obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        _run([HIPCC] + HIP_FLAGS + lang + ["-c", path, "-o", obj], verbose)
        objs.append(obj)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
