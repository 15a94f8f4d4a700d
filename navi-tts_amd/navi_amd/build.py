"""Builds the in-tree native libraries (gfx950 HIP library, host C++ library, tools).

Everything is compiled into navi-tts_amd/lib/ so it travels with the source tree
to the GPU box. No cmake/ninja: explicit hipcc/g++ lines, run in parallel.
"""
from __future__ import annotations

import os
import shlex
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent.parent          # navi-tts_amd/
ROOT = PKG.parent                                      # repo root
LIB = PKG / "lib"
OBJ = PKG / "lib" / "obj"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: no packed FP32 instructions (v_pk_*_f32) in any HIP code: some of their forms have
# given silently wrong results on this pool's MI355X boxes.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", str(ROOT / "include"), "-I", str(PKG / "csrc" / "hip")]

HIP_SOURCES = ["device.hip", "frame.hip", "prefill.hip", "vocoder.hip", "streams.hip", "speaker.hip"]
HOST_SOURCES = ["graph.cpp"]          # csrc/host: C++ over the C ABI, no device code
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-I", str(ROOT / "include")]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed ({r.returncode}): {' '.join(shlex.quote(c) for c in cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _newer(target: Path, deps: list[Path]) -> bool:
    return target.exists() and all(target.stat().st_mtime >= d.stat().st_mtime for d in deps)


def build_randinit() -> Path:
    LIB.mkdir(parents=True, exist_ok=True)
    out = LIB / "librandinit.so"
    _run(["gcc", "-O3", "-fopenmp", "-fPIC", "-shared", "-o", str(out), str(PKG / "tools" / "randinit.c"), "-lm"])
    return out


def build_hip(jobs: int = 8) -> Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    headers = list((PKG / "csrc" / "hip").glob("*.h")) + [ROOT / "include" / "navi_amd.h"]
    objs = []

    def compile_one(src: str) -> Path:
        s = PKG / "csrc" / "hip" / src
        o = OBJ / (src + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)])
        return o

    def compile_host(src: str) -> Path:
        o = OBJ / (src + ".o")
        _run(["g++", *HOST_FLAGS, "-c", str(PKG / "csrc" / "host" / src), "-o", str(o)])
        return o

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        hip = ex.map(compile_one, HIP_SOURCES)
        host = ex.map(compile_host, HOST_SOURCES)
        objs = list(hip) + list(host)
    out = LIB / "libnavi_amd.so"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(out), *map(str, objs)])
    return out


def build_bench() -> list[Path]:
    """The microbenchmarks behind the design's latency figures (standalone programs): the frame
    kernel's exchange hop, the dependent-launch floor of the row-projection chains, the cost
    of a grid-wide barrier phase in a persistent grid exchanging 32-row activations, how a
    poll's round trip grows with other waves' or its own wave's weight loads in flight, the read
    rate of the row projections' operand loads by memory layout, and the projections on the
    row-major and the tile layouts."""
    LIB.mkdir(parents=True, exist_ok=True)
    outs = []
    for name in ("hop_latency", "launch_floor", "grid_barrier", "load_coupling", "operand_layout", "row_tiles"):
        out = LIB / name
        _run([HIPCC, "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-I", str(ROOT / "include"), "-I", str(PKG / "csrc" / "hip"),
              "-o", str(out), str(PKG / "csrc" / "bench" / (name + ".hip"))])
        outs.append(out)
    return outs


def build_all() -> None:
    """The product: the HIP library and the random-init tool (the microbenchmarks are built on
    demand, `python -m navi_amd.build bench`)."""
    build_randinit()
    build_hip()


if __name__ == "__main__":
    if sys.argv[1:] == ["bench"]:
        build_bench()
    else:
        build_all()
