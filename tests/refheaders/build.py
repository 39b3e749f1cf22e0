"""Build recipe of the reference-header drivers (test infrastructure).

Compiles tests/refheaders/*_driver.cpp with g++ against the reference's own
model headers, read where they lie under /root/reference/src (included, not
copied), and this build's ggml API layer (minimaxmusic.cpp_amd/ggml/include),
linking libggml-base.so; the MI355X backend is loaded at run time by
ggml_backend_load_all as the reference does (src/backend.h:106).  Output:
tests/refheaders/_build/<name> (git-ignored; it travels with the tree to the
GPU machine, where the reference tree is absent).

    python tests/refheaders/build.py
"""
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REF_SRC = pathlib.Path("/root/reference/src")
GGML_INC = ROOT / "minimaxmusic.cpp_amd" / "ggml" / "include"
LIB = ROOT / "minimaxmusic.cpp_amd" / "lib"
OUT = HERE / "_build"
DRIVERS = ["lm_driver", "depth_driver", "dit_driver"]


def available():
    return (REF_SRC / "qwen3-lm.h").exists()


def build(verbose=False):
    if not available():
        raise RuntimeError(f"{REF_SRC} is not present: the drivers are built where the reference tree is")
    OUT.mkdir(exist_ok=True)
    built = []
    for name in DRIVERS:
        out = OUT / name
        cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
               f"-I{REF_SRC}", f"-I{GGML_INC}", str(HERE / f"{name}.cpp"), "-o", str(out) + ".tmp",
               f"-L{LIB}", "-lggml-base", "-ldl", "-Wl,-rpath,$ORIGIN/../../../minimaxmusic.cpp_amd/lib"]
        if verbose:
            print(" ".join(cmd))
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"build of {name} failed:\n{r.stderr}")
        pathlib.Path(str(out) + ".tmp").replace(out)
        built.append(out)
    return built


if __name__ == "__main__":
    for p in build(verbose="-v" in sys.argv):
        print(p)
