"""Build recipe for the MI355X (gfx950) shared libraries of this package.

    python -m build  (from this directory)   or   build.build_all()

Compiles the HIP sources with hipcc for gfx950 (and the host-only ggml core
with clang++) into _build/ and links, in-tree under lib/:
  libmmhip.so        the kernel C-ABI (include/mmhip.h)
  libggml-base.so    the restated ggml-base subset (ggml/include/*.h)
  libggml-mi355x.so  the MI355X ggml backend (include/ggml-mi355x.h)
  libmm_lm.so        the LM batched decode step on that backend (include/mm_lm.h)
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
CLANGXX = os.environ.get("CLANGXX", "/opt/rocm/llvm/bin/clang++")
ARCH = "gfx950"
GGML_INC = PKG / "ggml" / "include"

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
    f"-I{GGML_INC}",
]

HOST_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", f"-I{GGML_INC}", f"-I{ROOT / 'include'}"]

# (library, compiler, sources, link flags)
LIBS = [
    ("libmmhip.so", "hip",
     ["csrc/k_quant.hip", "csrc/k_gemv.hip", "csrc/k_gemm.hip", "csrc/k_fa_decode.hip", "csrc/k_fa_mfma.hip",
      "csrc/k_glue.hip", "csrc/k_synth.hip", "csrc/mmhip_api.hip"], []),
    # stand-in for libggml-base (ggml is not vendored by the reference)
    ("libggml-base.so", "host", ["ggml/src/ggml_core.cpp", "ggml/src/gguf.cpp"], ["-ldl"]),
    # the MI355X ggml backend, on top of the two above
    ("libggml-mi355x.so", "hip", ["csrc/ggml-mi355x.cpp"],
     ["-L{lib}", "-lmmhip", "-lggml-base", "-Wl,-rpath,$ORIGIN"]),
    # Qwen3-shape LM batched decode step built with the ggml API (include/mm_lm.h)
    ("libmm_lm.so", "hip", ["csrc/mm_lm.cpp"],
     ["-L{lib}", "-lggml-mi355x", "-lggml-base", "-lmmhip", "-Wl,-rpath,$ORIGIN"]),
]


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{errs}")
    if errs.strip() and verbose:
        print(errs, file=sys.stderr)


def _compile(kind, src, obj, verbose):
    if kind == "hip":
        cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [CLANGXX, *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    _run(cmd, f"compile {src.name}", verbose)


def build_all(verbose: bool = False, jobs: int = 8) -> list:
    BUILD.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    jobs_list = []
    for lib, kind, srcs, _ in LIBS:
        for s in srcs:
            src = PKG / s
            jobs_list.append((kind, src, BUILD / (src.stem + ".o")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_compile, k, s, o, verbose) for k, s, o in jobs_list]:
            f.result()
    built = []
    for lib, kind, srcs, ldflags in LIBS:
        objs = [str(BUILD / (pathlib.Path(s).stem + ".o")) for s in srcs]
        out = LIB / lib
        tmp = LIB / (lib + ".tmp")
        flags = [f.replace("{lib}", str(LIB)) for f in ldflags]
        if kind == "hip":
            cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp), *flags]
        else:
            cmd = [CLANGXX, "-shared", "-fPIC", *objs, "-o", str(tmp), *flags]
        _run(cmd, f"link {lib}", verbose)
        os.replace(tmp, out)
        built.append(out)
    return built


if __name__ == "__main__":
    for p in build_all(verbose="-v" in sys.argv):
        print(p)
