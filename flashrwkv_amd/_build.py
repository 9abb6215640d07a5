"""Build recipe for the in-tree native libraries.

* ``libflashrwkv_amd.so``: the HIP kernels and the C ABI of
  ``include/flashrwkv_amd.h``, compiled by ``hipcc --offload-arch=gfx950``.
* ``_flashrwkv_amd_ops.so``: the thin TORCH_LIBRARY binding, compiled by g++
  against the installed PyTorch-ROCm headers and linked to the library above.

No hipify step and no ``torch.utils.cpp_extension``: every source is written
for gfx950 directly. Run ``python -m flashrwkv_amd._build`` or
``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sysconfig
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
REPO = PKG.parent
LIB = PKG / "libflashrwkv_amd.so"
OPS = PKG / "_flashrwkv_amd_ops.so"
OBJ_DIR = PKG / "_build"

HIP_SOURCES = sorted(CSRC.glob("*.hip"))
BINDING_SOURCE = CSRC / "binding" / "torch_ops.cpp"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU ops stay disabled for all device code on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(REPO / "include"),
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


# Per-file scheduler choice. The chunk kernels are latency-bound at two waves
# per SIMD; LLVM's max-ilp strategy orders their MFMA/LDS chains for
# instruction-level parallelism instead of register pressure. Same-box A/B,
# results bitwise identical: backward 1.580 -> 1.556 ms (config 4), dense
# prefill 0.447 -> 0.440 ms (config 3), varlen unchanged.
FILE_FLAGS = {
    "chunk_fwd": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "chunk_bwd": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


def _compile_hip(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    _run([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src.stem, []), "-c", str(src), "-o", str(obj)])
    return obj


def build_library() -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as pool:
        objs = list(pool.map(_compile_hip, HIP_SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs),
          "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def _torch_paths() -> tuple[Path, Path]:
    import torch  # noqa: PLC0415

    root = Path(torch.__file__).resolve().parent
    return root / "include", root / "lib"


def build_binding() -> Path:
    inc, lib = _torch_paths()
    tmp = OPS.with_suffix(".so.tmp")
    _run([
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DFRWKV_PYTHON_MODULE=1",
        "-DTORCH_EXTENSION_NAME=_flashrwkv_amd_ops", "-I", sysconfig.get_paths()["include"],
        "-I", str(inc), "-I", str(inc / "torch" / "csrc" / "api" / "include"),
        "-I", "/opt/rocm/include", "-I", str(REPO / "include"),
        str(BINDING_SOURCE), "-o", str(tmp),
        "-L", str(PKG), "-lflashrwkv_amd",
        "-L", str(lib), "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_python",
        f"-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{lib}",
    ])
    os.replace(tmp, OPS)
    return OPS


# Host-side AddressSanitizer build of the library, for the CPU tests of the C
# ABI's host code (argument checks, workspace sizing, error reporting). The
# sanitizer flags reach the host compilation only (each behind -Xarch_host);
# the device code is built as usual (at -O1: it is never launched from this
# build, which runs where there is no GPU). Loaded by a process that preloads
# the matching runtime (asan_runtime()).
ASAN_DIR = OBJ_DIR / "asan"
ASAN_LIB = ASAN_DIR / "libflashrwkv_amd_asan.so"
ASAN_HOST_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
                   "-Xarch_host", "-g"]


def asan_runtime() -> Path | None:
    """The clang AddressSanitizer runtime that ASAN_LIB links against."""
    found = sorted(Path("/opt/rocm/lib/llvm/lib/clang").glob(
        "*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def _compile_hip_asan(src: Path) -> Path:
    obj = ASAN_DIR / (src.stem + ".o")
    flags = [f for f in HIP_FLAGS if f != "-O3"]
    _run([HIPCC, *flags, "-O1", *ASAN_HOST_FLAGS, "-c", str(src), "-o", str(obj)])
    return obj


def build_sanitized_library() -> Path:
    ASAN_DIR.mkdir(parents=True, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as pool:
        objs = list(pool.map(_compile_hip_asan, HIP_SOURCES))
    tmp = ASAN_LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
          "-shared-libasan", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, ASAN_LIB)
    return ASAN_LIB


def build() -> tuple[Path, Path]:
    """Compile every native artefact (always rebuilds)."""
    return build_library(), build_binding()


if __name__ == "__main__":
    for path in build():
        print(path)
    if "--asan" in sys.argv[1:]:
        print(build_sanitized_library())
