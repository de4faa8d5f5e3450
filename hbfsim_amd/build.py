"""Builds hbfsim_amd/libhbfsim_amd.so for gfx950 with hipcc.

The library is built in-tree so it travels with the repository to the GPU
host.  Device code is compiled without packed-FP32 instruction selection.
"""
from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
LIB = HERE / "libhbfsim_amd.so"

SOURCES = [CSRC / "engine.hip", CSRC / "gen.hip", CSRC / "thermal.hip", CSRC / "servers.hip",
           CSRC / "hybrid.hip", CSRC / "link.hip", CSRC / "admission.hip", CSRC / "order.hip",
           CSRC / "probe.hip", CSRC / "api.cpp",
           CSRC / "profile.cpp"]
HEADERS = [CSRC / "engine.hpp", CSRC / "thermal.hpp", CSRC / "link.hpp", CSRC / "profile.hpp",
           CSRC / "json_min.hpp", ROOT / "include" / "hbfsim_amd.h"]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and pathlib.Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: the HIP engine cannot be built")


FLAGS = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-fvisibility=hidden", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def command(output: pathlib.Path = LIB) -> list[str]:
    """The whole library in one hipcc call (kept for reference; build() runs
    the same flags per source in parallel, then links)."""
    return [hipcc(), *FLAGS, "-shared", "-I", str(ROOT / "include"), "-o", str(output),
            *[str(s) for s in SOURCES]]


def object_command(source: pathlib.Path, output: pathlib.Path) -> list[str]:
    return [hipcc(), *FLAGS, "-I", str(ROOT / "include"), "-c", "-o", str(output), str(source)]


def link_command(objects: list[pathlib.Path], output: pathlib.Path) -> list[str]:
    return [hipcc(), "--offload-arch=gfx950", "-fPIC", "-shared", "-o", str(output),
            *[str(o) for o in objects]]


CLI = HERE / "hbf_trace_timing"
CLI_SOURCES = [CSRC / "trace_timing.cpp", CSRC / "profile.cpp"]


def cli_command(output: pathlib.Path = CLI) -> list[str]:
    """The hbf_trace_timing drop-in: host code, linked against the library
    (its GPU sampler serves hybrid mode), found next to the executable."""
    return [hipcc(), "-O2", "-std=c++17", "-Wall", "-o", str(output),
            *[str(s) for s in CLI_SOURCES], "-L", str(HERE), "-lhbfsim_amd",
            "-Wl,-rpath,$ORIGIN"]


MEDIA_BENCH = HERE / "hbf_media_bench"
MEDIA_BENCH_SOURCES = [CSRC / "media_bench.cpp", CSRC / "profile.cpp"]


def media_bench_command(output: pathlib.Path = MEDIA_BENCH) -> list[str]:
    """hbf_media_bench: host code timing through the library."""
    return [hipcc(), "-O2", "-std=c++17", "-Wall", "-o", str(output),
            *[str(s) for s in MEDIA_BENCH_SOURCES], "-L", str(HERE), "-lhbfsim_amd",
            "-Wl,-rpath,$ORIGIN"]


def build_cli(verbose: bool = False) -> pathlib.Path:
    tmp = CLI.with_suffix(".tmp")
    cmd = cli_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"c++ failed with status {proc.returncode}")
    os.replace(tmp, CLI)
    tmp = MEDIA_BENCH.with_suffix(".tmp")
    _run(media_bench_command(tmp), verbose)
    os.replace(tmp, MEDIA_BENCH)
    return CLI


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with status {proc.returncode}: {cmd[-1]}")
    if verbose and proc.stderr.strip():
        sys.stderr.write(proc.stderr)


def build(verbose: bool = False) -> pathlib.Path:
    """Compiles every source every time it is called: one object per source
    (in parallel, at most 8 at a time), then one link."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    objects = [objdir / (src.name + ".o") for src in SOURCES]
    jobs = max(1, min(8, os.cpu_count() or 1, len(SOURCES)))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda so: _run(object_command(*so), verbose), zip(SOURCES, objects)))
    tmp = LIB.with_suffix(".so.tmp")
    _run(link_command(objects, tmp), verbose)
    os.replace(tmp, LIB)
    build_cli(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
