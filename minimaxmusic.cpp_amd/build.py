"""Build recipe for the MI355X (gfx950) shared libraries of this package.

    python -m build  (from this directory)   or   build.build_all()

Compiles every csrc/*.hip with hipcc for gfx950 into _build/, links
lib/libmmhip.so (the kernel C-ABI, include/mmhip.h) in-tree so that it
travels with the source tree.
"""
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-result",
    # packed fp32 instructions stay off: only scalar fp32 VALU ops are emitted
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]

LIBS = {
    "libmmhip.so": ["k_quant.hip", "k_gemv.hip", "k_gemm.hip", "k_fa_decode.hip", "k_fa_mfma.hip", "mmhip_api.hip"],
}


def _compile(src: pathlib.Path, obj: pathlib.Path, verbose: bool) -> None:
    cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{errs}")
    if errs.strip() and verbose:
        print(errs, file=sys.stderr)


def build_all(verbose: bool = False, jobs: int = 8) -> list:
    BUILD.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    built = []
    for lib, srcs in LIBS.items():
        objs = []
        with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
            futs = []
            for s in srcs:
                src = CSRC / s
                obj = BUILD / (src.stem + ".o")
                objs.append(obj)
                futs.append(ex.submit(_compile, src, obj, verbose))
            for f in futs:
                f.result()
        out = LIB / lib
        tmp = LIB / (lib + ".tmp")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link of {lib} failed:\n{r.stderr}")
        os.replace(tmp, out)
        built.append(out)
    return built


if __name__ == "__main__":
    for p in build_all(verbose="-v" in sys.argv):
        print(p)
