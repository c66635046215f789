"""Builds libartemis_sampler.so for gfx950 with hipcc, in-tree beside this file.

Every HIP source is compiled with -ffp-contract=off (no fused multiply-add except the ones the f64
exp writes explicitly), IEEE f32 division, and packed f32 arithmetic disabled. The sources compile to
objects in parallel (under _build/ beside this file), then link into the shared library.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libartemis_sampler.so")
SOURCES = ["api.hip", "scan.hip", "finish.hip", "misc.hip", "logprobs.hip", "embed.hip", "matvec.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    return r


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    objs = [os.path.join(OBJ, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[HIPCC, *FLAGS, "-c", "-o", o, os.path.join(CSRC, s)] for s, o in zip(SOURCES, objs)]
    jobs = max(1, min(len(cmds), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda c: _run(c, verbose), cmds))
    failed = [r for r in results if r.returncode != 0]
    for r in results:
        if r.stdout or r.stderr:
            sys.stderr.write(r.stdout + r.stderr)
    if failed:
        raise RuntimeError("hipcc failed compiling a source of libartemis_sampler.so")
    r = _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB + ".tmp", *objs], verbose)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed linking libartemis_sampler.so")
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
