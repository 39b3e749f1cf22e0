"""The C-ABI library loads and exports every function include/mmhip.h declares
(no compute calls: runs without a GPU)."""
import ctypes
import pathlib
import re

ROOT = pathlib.Path(__file__).resolve().parent.parent


def declared_functions(header):
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mmhip_[a-z0-9_]+)\s*\(", text)))


def declared(header, prefix):
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / header).read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(" + prefix + r"[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported(pkg):
    import __graft_entry__

    lib = pkg.mmhip.LIB_PATH
    if not lib.exists():
        __graft_entry__.build()
    L = ctypes.CDLL(str(lib))
    names = declared_functions(ROOT / "include" / "mmhip.h") + declared("mmhip_synth.h", "mmhip_")
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
        assert n in pkg.mmhip.SIGNATURES, f"{n} missing from the Python binding"


def test_backend_and_lm_symbols_exported(pkg):
    libdir = pkg.mmhip.LIB_PATH.parent
    base = ctypes.CDLL(str(libdir / "libggml-base.so"), mode=ctypes.RTLD_GLOBAL)
    be = ctypes.CDLL(str(libdir / "libggml-mi355x.so"))
    for n in declared("ggml-mi355x.h", "ggml_backend_"):
        assert hasattr(be, n), n
    # dynamic-loading entry points of a ggml backend
    assert hasattr(be, "ggml_backend_init") and hasattr(be, "ggml_backend_score")
    for n in ("ggml_backend_graph_compute", "ggml_backend_tensor_set", "ggml_gallocr_alloc_graph",
              "ggml_flash_attn_ext", "ggml_mul_mat", "ggml_backend_load_all"):
        assert hasattr(base, n), n
    lm = ctypes.CDLL(str(libdir / "libmm_lm.so"))
    names = declared("mm_lm.h", "mm_lm_")
    assert len(names) >= 12
    for n in names:
        assert hasattr(lm, n), n


def test_error_reporting_without_gpu(pkg):
    """Argument validation runs on the host and reports through last_error."""
    L = pkg.mmhip.load()
    rc = L.mmhip_mul_mat(8, None, 0, 0, 0, None, 0, 0, None, 0, None, 0, None)
    assert rc == pkg.mmhip.ERR_INVALID
    assert b"bad arguments" in L.mmhip_last_error()
    rc = L.mmhip_repack_rows(3, None, None, 1, 32, None)
    assert rc == pkg.mmhip.ERR_UNSUPPORTED
    assert L.mmhip_act_bytes(8, 4096, 2) >= 2 * 4096 + 4 * 2 * 128
    assert L.mmhip_act_bytes(12, 100, 2) == 0


def test_noalloc_attention_rejects_oversize_on_host(pkg):
    """mmhip_flash_attn_ext_noalloc refuses a shape whose workspace exceeds its
    8 MiB device array before any HIP call (a masked attention of 16384 query
    rows x 64 heads x 2: 16 MiB of prepass rows); the operand pointers are
    host addresses that are never dereferenced."""
    import numpy as np

    mm = pkg.mmhip
    L = mm.load()
    assert L.mmhip_flash_attn_noalloc_max_workspace() == 8 << 20
    buf = np.zeros(64, np.float32)
    base = buf.ctypes.data + (-buf.ctypes.data) % 16

    def view(ne, nb):
        v = mm.MmhipView()
        v.data = base
        v.ne[:] = list(ne)
        v.nb[:] = list(nb)
        return v

    D, nq, Hq, B, nkv = 64, 16384, 64, 2, 64
    q = view((D, nq, Hq, B), (4, 4 * D, 4 * D * nq, 4 * D * nq * Hq))
    k = view((D, nkv, 8, B), (2, 2 * D, 2 * D * nkv, 2 * D * nkv * 8))
    m = view((nkv, nq, 1, 1), (2, 2 * nkv, 2 * nkv * nq, 2 * nkv * nq))
    need = L.mmhip_flash_attn_workspace(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k))
    rc = L.mmhip_flash_attn_ext_noalloc(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), ctypes.byref(m), 0.125,
                                        ctypes.c_void_p(base), None)
    assert rc == mm.ERR_WORKSPACE, L.mmhip_last_error()
    assert b"maximum" in L.mmhip_last_error()
