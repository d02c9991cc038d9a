"""Build recipe for libw8a8_gfx950.so (hipcc, gfx950, in-tree).

``python -m nanopointllm_amd.build`` (with ``nano-pointllm_amd`` on
``sys.path``) compiles every ``csrc/*.hip`` translation unit in parallel and
links the shared library next to this file.  It also links the diagnostic
``libw8a8_gfx950_timeline.so``: the same objects with the fused decode
kernel rebuilt under ``W8A8_TIMELINE`` (per-workgroup start-up timestamps,
read back through ``w8a8_timeline_read``), which ``bench.py
--profile-timeline`` loads.  The library proper contains none of it.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent                      # nano-pointllm_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"          # repository include/ (public C header)
BUILD_DIR = ROOT / "_build"
LIB_NAME = "libw8a8_gfx950.so"
LIB_PATH = PKG_DIR / LIB_NAME
TIMELINE_LIB_PATH = PKG_DIR / "libw8a8_gfx950_timeline.so"
TIMELINE_SOURCE = "gemv_fused.hip"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the W8A8 HIP library cannot be built")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-fno-gpu-rdc",
        # The dequant epilogue needs separate binary32 roundings.
        "-ffp-contract=off",
        # Keep the compiler from emitting packed-FP32 VALU ops.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-result",
        f"-I{CSRC}",
        f"-I{INCLUDE}",
    ]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, timeline: bool = False) -> Path:
    obj = BUILD_DIR / (src.stem + ("_timeline" if timeline else "") + ".o")
    defs = ["-DW8A8_TIMELINE=1"] if timeline else []
    cmd = [hipcc(), *compile_flags(), *defs, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile all translation units and link ``libw8a8_gfx950.so``."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = [(src, False) for src in srcs]
    jobs += [(src, True) for src in srcs if src.name == TIMELINE_SOURCE]
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda job: _compile(*job), jobs))
    plain = [o for o, (_, tl) in zip(objs, jobs) if not tl]
    timeline = [o for o, (src, tl) in zip(objs, jobs)
                if tl or (src.name != TIMELINE_SOURCE)]
    for path, group in ((LIB_PATH, plain), (TIMELINE_LIB_PATH, timeline)):
        _link(path, group)
        if verbose:
            print(f"built {path}", file=sys.stderr)
    return LIB_PATH


def _link(path: Path, objs: list[Path]) -> None:
    tmp = path.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, path)


if __name__ == "__main__":
    build(verbose=True)
