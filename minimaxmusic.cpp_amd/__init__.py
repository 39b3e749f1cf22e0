"""MI355X-native (gfx950) ggml backend pieces for minimaxmusic.cpp's attention
and quantized-matmul hot path.

The product is native: HIP kernels behind the C-ABI in include/mmhip.h
(lib/libmmhip.so).  This Python package is the host mirror used by tests and
the benchmark: ``mmhip`` binds the C-ABI, ``synth`` makes the seeded synthetic
inputs, ``build`` compiles the libraries in-tree.

The directory name contains a dot, so load it by path, e.g. with
``importlib.util.spec_from_file_location("mmcpp_amd", <dir>/__init__.py,
submodule_search_locations=[<dir>])``.
"""
from . import mmhip, synth  # noqa: F401
