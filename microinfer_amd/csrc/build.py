"""Build libmi_attn.so (gfx950) from the HIP sources in this directory.

Usage: ``python -m microinfer_amd.csrc.build`` or ``build()`` from Python.
Every ``*.hip`` here is compiled to an object under ``microinfer_amd/_build``
(in parallel) and linked into ``microinfer_amd/libmi_attn.so``. Always
recompiles: the caller asked for a build.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PACKAGE = CSRC.parent
REPO = PACKAGE.parent
BUILD_DIR = PACKAGE / "_build"
LIBRARY = PACKAGE / "libmi_attn.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Keep the compiler from forming packed-fp32 VALU ops.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


def _compile(source: Path, build_dir: Path, extra_flags: tuple[str, ...]) -> Path:
    obj = build_dir / (source.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *extra_flags, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = False, *, extra_flags: tuple[str, ...] = (),
          output: Path | None = None) -> Path:
    """Compile and link; ``extra_flags``/``output`` build a variant library."""
    library = LIBRARY if output is None else Path(output)
    build_dir = BUILD_DIR if output is None else library.parent / (library.stem + "_build")
    build_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), max(1, min(16, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(lambda s: _compile(s, build_dir, tuple(extra_flags)), sources))
    tmp = library.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, library)
    if verbose:
        print(f"built {library} from {len(sources)} sources", file=sys.stderr)
    return library


if __name__ == "__main__":
    build(verbose=True)
