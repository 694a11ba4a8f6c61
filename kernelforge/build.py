"""Build libkernelforge_hip.so for gfx950, in-tree.

    python -m kernelforge.build [--jobs N]

Steps:
1. Generate the GEMM instantiation list from the search space's
   shape-independent rules (:func:`kernelforge.tuning.search.gemm_instantiations`),
   split into chunks so the translation units compile in parallel.
2. ``hipcc --offload-arch=gfx950 -c`` every translation unit.
3. Link ``kernelforge/libkernelforge_hip.so``.

Always recompiles: a stale library must never pass for the current sources.
"""

from __future__ import annotations

import argparse
import hashlib
import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
REPO = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = REPO / "include"
BUILD = REPO / "_build"
GEN = BUILD / "gen"
LIBRARY = PACKAGE / "libkernelforge_hip.so"

OFFLOAD_ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

#: hipcc flags for every translation unit. Packed-fp32 VALU ops are disabled:
#: their hand-written forms are avoided on these boxes and the compiler must
#: not form them either.
HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]

#: Tiles per GEMM translation unit.
TILES_PER_CHUNK = 8

#: (dtype code, element bytes); codes match KF_DTYPE_* in include/kernelforge_hip.h.
DTYPES = ((0, 4), (1, 2), (2, 2))
#: Loader pairs: 0 = VecK/VecN, 1 = VecK/VecK, 2 = Scalar/Scalar (register-staged
#: pipeline); 3 = DMA with n-contiguous B, 4 = DMA with k-contiguous B (direct).
COMBOS = (0, 1, 2, 3, 4)
DIRECT_COMBOS = (3, 4)


def generate() -> list[tuple[int, int, int, Path]]:
    """Write the tile lists and the registry include; return the GEMM units."""
    sys.path.insert(0, str(REPO))
    from kernelforge.tuning.search import gemm_instantiations

    GEN.mkdir(parents=True, exist_ok=True)
    staged = gemm_instantiations(direct=0)
    direct = gemm_instantiations(direct=1)
    units = []
    registry = []
    for dt, elem in DTYPES:
        for combo in COMBOS:
            lst = (direct if combo in DIRECT_COMBOS else staged)[elem]
            chunks = [lst[i : i + TILES_PER_CHUNK] for i in range(0, len(lst), TILES_PER_CHUNK)]
            for c, chunk in enumerate(chunks):
                inc = GEN / f"gemm_tiles_{dt}_{combo}_{c}.inc"
                inc.write_text("".join(f"KF_VARIANT({bm}, {bn}, {bk}, {w}, {s})\n" for bm, bn, bk, w, s in chunk))
                units.append((dt, combo, c, inc))
                registry.append(f"KF_TABLE({dt}, {combo}, {c})\n")
    (GEN / "gemm_tables.inc").write_text("".join(registry))
    return units


def source_digest() -> str:
    """First 16 hex digits of SHA-256 over everything a build compiles: the
    sources under csrc/ and include/, the GEMM tile lists the search space
    generates, and the compiler flags. Built into the library
    (``kf_source_digest``), so a profile or measurement can name the exact
    code it ran, and identical for every rebuild of the same tree."""
    sys.path.insert(0, str(REPO))
    from kernelforge.tuning.search import gemm_instantiations

    h = hashlib.sha256()
    for path in sorted([*CSRC.iterdir(), *INCLUDE.glob("*.h")]):
        if path.is_file():
            h.update(path.name.encode() + b"\0" + path.read_bytes() + b"\0")
    for direct in (0, 1):
        h.update(repr(sorted(gemm_instantiations(direct=direct).items())).encode())
    h.update(" ".join(HIP_FLAGS).encode())
    return h.hexdigest()[:16]


def _compile(src: Path, obj: Path, extra: list[str]) -> tuple[Path, float, str]:
    t0 = time.perf_counter()
    cmd = [HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", f"-I{GEN}", *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature; that warning is noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    log = "\n".join(l for l in (proc.stdout + proc.stderr).splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name} {' '.join(extra)}:\n{log}")
    return obj, time.perf_counter() - t0, log


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    jobs = jobs or min(16, os.cpu_count() or 1)
    t0 = time.perf_counter()
    obj_dir = BUILD / "obj"
    if obj_dir.exists():
        shutil.rmtree(obj_dir)
    obj_dir.mkdir(parents=True)
    units = generate()
    digest = source_digest()
    tasks = [
        (CSRC / "abi.hip", obj_dir / "abi.o", [f'-DKF_SOURCE_DIGEST="{digest}"']),
        (CSRC / "rows.hip", obj_dir / "rows.o", []),
        (CSRC / "gemv.hip", obj_dir / "gemv.o", []),
        (CSRC / "wide_rows.hip", obj_dir / "wide_rows.o", []),
        (CSRC / "elementwise.hip", obj_dir / "elementwise.o", []),
        (CSRC / "gemm.hip", obj_dir / "gemm.o", []),
    ]
    for dt, combo, c, inc in units:
        tasks.append(
            (
                CSRC / "gemm_inst.hip",
                obj_dir / f"gemm_{dt}_{combo}_{c}.o",
                [f"-DKF_DT={dt}", f"-DKF_COMBO={combo}", f"-DKF_CHUNK={c}", f'-DKF_TILES_INC="{inc.name}"'],
            )
        )
    # Longest first: the GEMM units dominate.
    tasks.sort(key=lambda t: 0 if t[0].name == "gemm_inst.hip" else 1)
    objs = []
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for obj, secs, log in pool.map(lambda t: _compile(*t), tasks):
            objs.append(obj)
            if log.strip() and verbose:
                print(log, file=sys.stderr)
    tmp = LIBRARY.with_suffix(".so.tmp")
    link = [HIPCC, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(
            f"built {LIBRARY.relative_to(REPO)} (sources {digest}): {len(tasks)} units "
            f"({len(units)} GEMM chunks) in {time.perf_counter() - t0:.1f}s with {jobs} jobs"
        )
    return LIBRARY


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--jobs", type=int, default=None)
    args = parser.parse_args(argv)
    build(args.jobs)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
