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


def test_header_symbols_exported(pkg):
    import __graft_entry__

    lib = pkg.mmhip.LIB_PATH
    if not lib.exists():
        __graft_entry__.build()
    L = ctypes.CDLL(str(lib))
    names = declared_functions(ROOT / "include" / "mmhip.h")
    assert len(names) >= 12
    for n in names:
        assert hasattr(L, n), n
        assert n in pkg.mmhip.SIGNATURES, f"{n} missing from the Python binding"


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
