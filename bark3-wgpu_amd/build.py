"""Build recipe for libbark_hip.so and libbark_hip.a (gfx950) — run by
__graft_entry__.build().

Each csrc/*.hip is compiled separately (in parallel) with hipcc for gfx950.
The objects are linked into bark3-wgpu_amd/libbark_hip.so, which the Python
host layer loads with ctypes, and archived into bark3-wgpu_amd/libbark_hip.a,
the static library a Rust build.rs links (with amdhip64 and the C++ runtime:
`-lamdhip64 -lstdc++`; each object carries its own gfx950 code object, so no
device link step is needed). Packed-FP32 instructions are disabled for device
code (-packed-fp32-ops); hipcc's host pass prints a harmless warning about it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libbark_hip.so"
STATIC = PKG / "libbark_hip.a"
ARCH = os.environ.get("BARK_HIP_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    tmp_a = STATIC.with_suffix(".a.tmp")
    if tmp_a.exists():
        tmp_a.unlink()
    r = subprocess.run(["ar", "rcs", str(tmp_a), *map(str, objs)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ar failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp_a, STATIC)
    if verbose:
        print(f"built {LIB} and {STATIC.name} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
