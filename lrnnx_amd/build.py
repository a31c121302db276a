"""Build liblrnnx_scan.so (gfx950) from lrnnx_amd/csrc with hipcc.

    python -m lrnnx_amd.build            # incremental (object newer than sources)
    python -m lrnnx_amd.build --force    # rebuild everything

Translation units are compiled in parallel; objects go to lrnnx_amd/_build/
and the shared library to lrnnx_amd/liblrnnx_scan.so (both git-ignored; the
.so travels with the tree to the GPU box).
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "liblrnnx_scan.so"
ARCH = os.environ.get("LRNNX_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

CFLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # packed FP32 (v_pk_*_f32) stays off on this hardware pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
    f"-I{ROOT / 'include'}",
    "-Wno-unused-command-line-argument",
]


def _sources():
    return sorted(CSRC.glob("*.hip"))


def _deps(src: Path) -> set[Path]:
    """Files `src` includes with #include "...", followed recursively."""
    seen: set[Path] = set()
    todo = [src]
    while todo:
        f = todo.pop()
        for line in f.read_text().splitlines():
            line = line.strip()
            if not line.startswith("#include") or '"' not in line:
                continue
            dep = (f.parent / line.split('"')[1]).resolve()
            if dep.exists() and dep not in seen:
                seen.add(dep)
                todo.append(dep)
    return seen


def _compile(src: Path, force: bool) -> tuple[Path, float, str]:
    obj = BUILD / (src.stem + ".o")
    newest_dep = max([src.stat().st_mtime] + [h.stat().st_mtime for h in _deps(src)])
    if not force and obj.exists() and obj.stat().st_mtime >= newest_dep:
        return obj, 0.0, ""
    t = time.time()
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops' is not a recognized" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")
    return obj, time.time() - t, msg


def build(force: bool = False, jobs: int | None = None, verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 1), 16)
    t0 = time.time()
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(lambda s: _compile(s, force), srcs))
    objs = [o for o, _, _ in results]
    relink = force or not LIB.exists() or any(o.stat().st_mtime > LIB.stat().st_mtime for o in objs)
    if relink:
        tmp = LIB.with_suffix(".so.tmp")
        cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objs), "-o", str(tmp)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
        os.replace(tmp, LIB)
    if verbose:
        for (o, dt, msg), s in zip(results, srcs):
            if dt:
                print(f"  compiled {s.name:28s} {dt:6.1f}s", flush=True)
            if msg.strip():
                print(msg, flush=True)
        print(f"built {LIB} in {time.time() - t0:.1f}s", flush=True)
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    a = ap.parse_args(argv)
    build(force=a.force, jobs=a.jobs)


if __name__ == "__main__":
    sys.exit(main())
