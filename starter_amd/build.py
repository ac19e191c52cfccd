"""Build the engine's native libraries in-tree (``starter_amd/_lib/``).

* ``libq3.so``     -- the gfx950 HIP kernels and their C-ABI launchers
                      (``csrc/*.hip``), built with ``hipcc --offload-arch=gfx950``.
* ``libq3seed.so`` -- the seeded-checkpoint generator (``csrc/seeded_init.c``),
                      plain C with OpenMP, built with ``gcc``.

Run ``python -m starter_amd.build``.  hipcc cross-compiles without a GPU.
"""

from __future__ import annotations

import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "_lib"
INCLUDE = HERE.parent / "include"

HIP_SOURCES = sorted(CSRC.glob("*.hip"))

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed FP32 (v_pk_*_f32) is kept out of the generated code on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{INCLUDE}",
]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [ln for ln in proc.stdout.splitlines()
             if "packed-fp32-ops' is not a recognized feature" not in ln]
    if lines:
        print("\n".join(lines), flush=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed ({proc.returncode}): {' '.join(cmd)}")


def build_seed_lib() -> pathlib.Path:
    OUT.mkdir(exist_ok=True)
    target = OUT / "libq3seed.so"
    tmp = OUT / "libq3seed.so.tmp"
    # No -ffast-math and no -march: the stream must be bit-identical on every
    # x86-64 host that runs this same binary.
    _run(["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-ffp-contract=off",
          str(CSRC / "seeded_init.c"), "-o", str(tmp), "-lm"])
    os.replace(tmp, target)
    return target


def build_hip_lib() -> pathlib.Path:
    """Compile each .hip file to an object in parallel, then link one shared library."""
    from concurrent.futures import ThreadPoolExecutor

    OUT.mkdir(exist_ok=True)
    objdir = OUT / "obj"
    objdir.mkdir(exist_ok=True)
    target = OUT / "libq3.so"
    tmp = OUT / "libq3.so.tmp"
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    objs = [objdir / (src.stem + ".o") for src in HIP_SOURCES]
    jobs = min(len(HIP_SOURCES), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda so: _run([hipcc, *compile_flags, "-c", str(so[0]), "-o", str(so[1])]),
                      zip(HIP_SOURCES, objs)))
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, target)
    return target


def build_all() -> None:
    build_seed_lib()
    if HIP_SOURCES:
        build_hip_lib()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
