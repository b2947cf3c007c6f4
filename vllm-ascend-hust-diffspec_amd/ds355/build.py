"""Build libds355.so in-tree with hipcc for gfx950.

``python -m ds355.build`` (or ``build()``) compiles every ``csrc/*.hip`` into
``ds355/libds355.so``: one hipcc process per source file, in parallel, into
a temporary directory, then one link.  The GPU code is built for gfx950 only,
with fp contraction off (the RoPE rotate must round each product separately),
packed-fp32 instructions disabled and the wave-level atomic aggregation off.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR.parent / "csrc"
LIBRARY = PACKAGE_DIR / "libds355.so"
ARCH = "gfx950"


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: the ds355 HIP library cannot be built")


def sources() -> list[Path]:
    return sorted(SOURCE_DIR.glob("*.hip"))


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # Keep single-lane atomics as written: the optimizer's wave-wide
        # aggregation reads the result back at once, which stalls a wave on
        # a device-scope round trip that the kernels hide behind their loads.
        "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
        "-Wall",
        "-Wno-unused-function",
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise subprocess.CalledProcessError(result.returncode, cmd, result.stdout, stderr)
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile the library; raises CalledProcessError with hipcc's output on failure."""
    tmp = LIBRARY.with_suffix(".so.tmp")
    srcs = sources()
    jobs = max(1, min(len(srcs), os.cpu_count() or 1, 16))
    with tempfile.TemporaryDirectory(prefix="ds355-build-") as work:
        objects = [Path(work) / (src.stem + ".o") for src in srcs]
        compiles = [[hipcc(), *flags(), "-c", "-o", str(obj), str(src)] for src, obj in zip(srcs, objects)]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            for future in [pool.submit(_run, cmd, verbose) for cmd in compiles]:
                future.result()
        _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *[str(o) for o in objects]], verbose)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    try:
        path = build(verbose=True)
    except subprocess.CalledProcessError as error:
        print(error.stderr, file=sys.stderr)
        sys.exit(error.returncode)
    print(path)
