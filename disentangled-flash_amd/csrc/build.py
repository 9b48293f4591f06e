"""Build ``libdflash.so`` for gfx950 with hipcc (no torch extension machinery).

Every ``*.hip`` file in this directory is compiled to an object in parallel,
then linked into ``disentangled_flash/libdflash.so`` next to the Python package
so the in-tree library travels with the source tree.

    python disentangled-flash_amd/csrc/build.py [--jobs N] [--verbose]
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PACKAGE_ROOT = CSRC.parent
REPO_ROOT = PACKAGE_ROOT.parent
INCLUDE = REPO_ROOT / "include"
OUTPUT = PACKAGE_ROOT / "disentangled_flash" / "libdflash.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU instructions.
# -unaligned-access-mode: keep the compiler from merging 2-byte LDS reads into
# unaligned 8-byte ones, which stall the LDS pipeline on gfx950.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=fast",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xclang", "-target-feature", "-Xclang", "-unaligned-access-mode",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return found


def _run(command: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(command)}\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False, output: Path = OUTPUT) -> Path:
    _build_library(sorted(CSRC.glob("*.hip")), output, jobs, verbose)
    return output


def _build_library(sources: list[Path], output: Path, jobs: int | None, verbose: bool) -> None:
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    compiler = hipcc()
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    with tempfile.TemporaryDirectory(prefix="dflash_build_") as tmp:
        objects = [Path(tmp) / (src.stem + ".o") for src in sources]
        commands = [
            [compiler, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
            for src, obj in zip(sources, objects)
        ]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            for future in [pool.submit(_run, cmd, verbose) for cmd in commands]:
                future.result()
        staged = Path(tmp) / output.name
        _run(
            [compiler, f"--offload-arch={ARCH}", "-shared", "-fPIC",
             *map(str, objects), "-o", str(staged)],
            verbose,
        )
        output.parent.mkdir(parents=True, exist_ok=True)
        shutil.move(str(staged), str(output))


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=None)
    parser.add_argument("--verbose", action="store_true")
    args = parser.parse_args()
    path = build(jobs=args.jobs, verbose=args.verbose)
    print(f"built {path}")


if __name__ == "__main__":
    main()
