"""Build recipe for the gfx950 C-ABI library ``libmi_amd.so``.

Compiles every ``csrc/*.hip`` file with hipcc for ``--offload-arch=gfx950`` and
links them into ``libmi_amd.so`` next to this file.  Objects are compiled in
parallel into ``_build/`` and relinked on every call (the driver's build check
compiles from scratch each round; ``force=False`` skips up-to-date objects).

Usage: ``python minimal-inference_amd/build.py [--force]``.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libmi_amd.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{CSRC}",
    f"-I{REPO_ROOT / 'include'}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _headers_mtime() -> float:
    hdrs = list(CSRC.glob("*.h")) + list((REPO_ROOT / "include").glob("*.h"))
    return max((h.stat().st_mtime for h in hdrs), default=0.0)


def _compile(hipcc: str, src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return obj, err


def build(force: bool = True, verbose: bool = False) -> Path:
    """Compile all kernels and link ``libmi_amd.so``; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = _sources()
    if not srcs:
        raise RuntimeError(f"no .hip sources under {CSRC}")
    hdr_t = _headers_mtime()
    jobs = []
    for src in srcs:
        obj = BUILD_DIR / (src.stem + ".o")
        stale = force or not obj.exists() or obj.stat().st_mtime < max(src.stat().st_mtime, hdr_t)
        jobs.append((src, obj, stale))
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "8")), 16))
    with cf.ThreadPoolExecutor(workers) as ex:
        futs = [ex.submit(_compile, hipcc, s, o) for s, o, stale in jobs if stale]
        for f in futs:
            obj, warn = f.result()
            if verbose and warn.strip():
                print(f"[{obj.name}] {warn}", file=sys.stderr)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp)]
    cmd += [str(o) for _, o, _ in jobs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(force=a.force, verbose=a.verbose))
