"""Builds libonpu_hip.so in-tree (opennpu_amd/libonpu_hip.so) with hipcc for gfx950, and the
benchmark's ceiling probes (opennpu_amd/libonpu_probe.so, csrc/onpu_probe.hip; no part of the ABI).

    python -m opennpu_amd.build          # or __graft_entry__.build()

Each source compiles to its own object in parallel, then one shared library is linked. All HIP
code is built with the packed-FP32 target feature off.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
OUT = HERE / "libonpu_hip.so"
PROBE = HERE / "libonpu_probe.so"
BUILD = HERE / "_build"
ARCH = os.environ.get("ONPU_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# (source, extra defines, object name): onpu_fmt.hip is built once per weight format
SOURCES = [("onpu_kernels.hip", [], "onpu_kernels"), ("onpu_codec.hip", [], "onpu_codec"), ("onpu_attn.hip", [], "onpu_attn"), ("onpu_api.cpp", [], "onpu_api"), ("onpu_quant.cpp", [], "onpu_quant")] + \
    [("onpu_fmt.hip", [f"-DONPU_FMT_ID={i}"], f"onpu_fmt{i}") for i in range(4)]
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", str(CSRC), "-I", str(ROOT / "include"),
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


def _compile(job):
    src, defs, name = job
    obj = BUILD / (name + ".o")
    cmd = [HIPCC, *FLAGS, *defs, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj


def build(verbose=True):
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(min(len(SOURCES) + 1, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES + [("onpu_probe.hip", [], "onpu_probe")]))
    probe = objs.pop()
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    tmp = PROBE.with_suffix(".so.tmp")
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), str(probe)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"probe link failed:\n{r.stderr}")
    os.replace(tmp, PROBE)
    if verbose:
        print(f"built {OUT} ({OUT.stat().st_size} bytes), {PROBE.name}")
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
