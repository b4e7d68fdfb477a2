"""Builds libanehip.so (all HIP sources in csrc/) for gfx950 with hipcc,
libane_engine.so (the C++ host API in engine/, over libanehip) with g++, and
libanehip_probe.so (bench/: the measurement-only roofline probes bench.py
loads, over libanehip).

Usage: python ane-infer_amd/build.py
The libraries are written next to this file so they travel with the source tree.
"""
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libanehip.so")
ENGINE_LIB = os.path.join(HERE, "libane_engine.so")
PROBE_LIB = os.path.join(HERE, "libanehip_probe.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

OBJ_DIR = os.path.join(HERE, "_build")

HIPCC_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++17",
    "-fPIC",
    # no packed fp32 instructions (v_pk_{add,mul,fma}_f32) in any kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))


def _run(cmd, what):
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    errs = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if res.returncode != 0:
        raise RuntimeError(f"{what} failed:\n" + "\n".join(errs))
    return errs


def build(verbose: bool = False) -> str:
    """Compiles every csrc/*.hip to an object (in parallel), links
    libanehip.so, then builds libane_engine.so."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(OBJ_DIR, os.path.basename(f)[:-4] + ".o") for f in srcs]
    cmds = [[hipcc, *HIPCC_FLAGS, "-c", "-o", o, f] for f, o in zip(srcs, objs)]
    if verbose:
        for c in cmds:
            print(" ".join(c), flush=True)
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as ex:
        warns = list(ex.map(lambda c: _run(c, "hipcc " + os.path.basename(c[-1])), cmds))
    for w in warns:
        if w and verbose:
            print("\n".join(w), file=sys.stderr)
    tmp = LIB + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs], "link")
    os.replace(tmp, LIB)
    build_engine(verbose)
    build_probe(hipcc, verbose)
    return LIB


def build_probe(hipcc: str, verbose: bool = False) -> str:
    """The measurement-only probe library (bench/probe.hip), linked to libanehip."""
    tmp = PROBE_LIB + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, "-shared", "-o", tmp, os.path.join(HERE, "bench", "probe.hip"), f"-L{HERE}",
           "-lanehip", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    _run(cmd, "hipcc probe.hip")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build_engine(verbose: bool = False) -> str:
    tmp = ENGINE_LIB + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra",
           f"-I{INCLUDE}", os.path.join(HERE, "engine", "ane_engine.cpp"), os.path.join(HERE, "engine", "gguf.cpp"),
           f"-L{HERE}", "-lanehip",
           "-Wl,-rpath,$ORIGIN", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("g++ failed:\n" + res.stderr)
    os.replace(tmp, ENGINE_LIB)
    return ENGINE_LIB


if __name__ == "__main__":
    print(build(verbose=True))
