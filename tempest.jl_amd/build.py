"""Build libtempest_hip.so for gfx950, in-tree, from csrc/*.hip.

Each source compiles to an object beside it under csrc/_obj, in parallel, and
the objects link into tempest.jl_amd/libtempest_hip.so.  Every build compiles
every source: this is the "does it build" check as well as the build.

    python tempest.jl_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJ = CSRC / "_obj"
LIB = HERE / "libtempest_hip.so"
INCLUDE = HERE.parent / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
    # No packed FP32 instructions: compile plain float code to scalar VALU.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-source extra flags.  The attention kernels keep their matrix-core
# accumulators in ordinary VGPRs (the VALU works on the scores directly, with
# no copies out of the accumulation registers).
EXTRA = {
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


# The check build: AddressSanitizer and UndefinedBehaviorSanitizer on the host
# code alone (the device code compiles as usual, uninstrumented), for the CPU
# tests of what the library does without a device (the floor's validation,
# planning, source writing, hiprtc and the code-object store).
SAN_FLAGS = ("-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined "
             "-Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer").split()


def sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: pathlib.Path) -> tuple[pathlib.Path, str]:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature; its warning is noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    out = "\n".join(l for l in (p.stdout + p.stderr).splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{out}")
    return obj, out


def build(jobs: int | None = None, verbose: bool = False) -> pathlib.Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, srcs))
    for obj, out in results:
        if out.strip() and verbose:
            print(out, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    # hiprtc compiles the generated floor kernels at run time.
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o, _ in results], "-lhiprtc"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stdout}{p.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_sanitized(dest: pathlib.Path, jobs: int | None = None) -> pathlib.Path:
    """The sanitized check library, built under `dest` (objects and
    libtempest_hip.so).  Load it with TEMPEST_HIP_LIBRARY set to its path and
    the sanitizer runtime preloaded (sanitizer_runtime())."""
    dest = pathlib.Path(dest)
    (dest / "obj").mkdir(parents=True, exist_ok=True)
    lib = dest / "libtempest_hip.so"

    def one(src: pathlib.Path) -> pathlib.Path:
        obj = dest / "obj" / (src.stem + ".o")
        cmd = [HIPCC, *FLAGS, *EXTRA.get(src.name, []), *SAN_FLAGS, "-Xarch_host", "-O1", "-Xarch_host", "-g",
               "-c", str(src), "-o", str(obj)]
        p = subprocess.run(cmd, capture_output=True, text=True)
        if p.returncode != 0:
            raise RuntimeError(f"hipcc (sanitized host) failed on {src.name}:\n{p.stdout}{p.stderr}")
        return obj

    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=jobs or min(len(srcs), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(one, srcs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libsan", *SAN_FLAGS, "-o", str(lib),
           *map(str, objs), "-lhiprtc"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{p.stdout}{p.stderr}")
    return lib


def sanitizer_runtime() -> pathlib.Path:
    """The AddressSanitizer runtime the sanitized library links against (the
    ROCm clang's own), to preload: python itself is not instrumented."""
    clang = pathlib.Path(HIPCC).resolve().parent / "../llvm/bin/clang"
    if not clang.exists():
        clang = pathlib.Path("/opt/rocm/llvm/bin/clang")
    out = subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                         text=True, check=True).stdout.strip()
    path = pathlib.Path(out)
    if not path.is_absolute() or not path.exists():
        raise RuntimeError(f"no AddressSanitizer runtime found ({out!r})")
    return path


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--sanitize", metavar="DIR", default=None,
                    help="build only the host-sanitized (ASan + UBSan) check library, under DIR")
    a = ap.parse_args()
    print(build_sanitized(pathlib.Path(a.sanitize), a.jobs) if a.sanitize else build(a.jobs, a.verbose))


if __name__ == "__main__":
    main()
