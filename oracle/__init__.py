"""ctypes binding of the CPU oracle (oracle.c) - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path (the HIP library and the ggml backend) never
does.  See oracle.h for what each function restates and oracle.c for how each
is pinned.
"""
import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, I32, I64, BF16 = 0, 1, 8, 12, 13, 14, 15, 26, 27, 30

BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292)}


def row_size(t, ne0):
    be, bb = BLOCK[t]
    assert ne0 % be == 0
    return ne0 // be * bb


def build(force=False):
    """Compile liboracle.so with the Makefile beside this file."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < max(
        (HERE / "oracle.c").stat().st_mtime, (HERE / "oracle.h").stat().st_mtime
    ):
        subprocess.run(["make", "-s", "-C", str(HERE), "-B" if force else "liboracle.so"], check=True)
    return LIB_PATH


class OrcTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
        L.orc_fp32_to_fp16.argtypes = [f32]
        L.orc_fp32_to_fp16.restype = ctypes.c_uint16
        L.orc_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.orc_fp16_to_fp32.restype = f32
        L.orc_fp32_to_bf16.argtypes = [f32]
        L.orc_fp32_to_bf16.restype = ctypes.c_uint16
        L.orc_fp32_to_fp16_row.argtypes = [vp, vp, i64]
        L.orc_fp16_to_fp32_row.argtypes = [vp, vp, i64]
        L.orc_dequantize_row.argtypes = [i32, vp, vp, i64]
        L.orc_quantize_row_q8_0.argtypes = [vp, vp, i64]
        L.orc_quantize_row_q8_K.argtypes = [vp, vp, i64]
        L.orc_vec_dot.argtypes = [i32, i64, vp, vp]
        L.orc_vec_dot.restype = f32
        L.orc_mul_mat_ggml.argtypes = [i32, vp, i64, i64, vp, i64, i64, vp, i32]
        L.orc_mul_mat_f64.argtypes = [i32, vp, i64, i64, vp, i64, i64, vp, i32]
        T = ctypes.POINTER(OrcTensor)
        L.orc_flash_attn_ext_ggml.argtypes = [T, T, T, T, f32, vp, i32]
        L.orc_flash_attn_ext_f64.argtypes = [T, T, T, T, f32, vp, i32]
        L.orc_rms_norm_mul.argtypes = [vp, vp, vp, i64, i64, f32]
        L.orc_layer_norm.argtypes = [vp, vp, i64, i64, f32]
        L.orc_rope_neox.argtypes = [vp, vp, i64, i64, i64, i64, vp, f32]
        L.orc_swiglu.argtypes = [vp, vp, i64, i64]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def default_threads():
    """Threads the restatement uses: the CPUs this process may run on (its
    affinity mask), capped by OMP_NUM_THREADS when that is set."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


# ---- conversions ----
def fp32_to_fp16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_fp32_to_fp16_row(_p(x), _p(y), x.size)
    return y


def fp16_bits_to_fp32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().orc_fp16_to_fp32_row(_p(h), _p(y), h.size)
    return y


# ---- block formats ----
def dequantize(t, blocks, ne0, nrows=1):
    """blocks: uint8 array of nrows * row_size(t, ne0) bytes -> f32 [nrows, ne0]."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    rs = row_size(t, ne0)
    assert blocks.size == rs * nrows
    out = np.empty((nrows, ne0), dtype=np.float32)
    for r in range(nrows):
        lib().orc_dequantize_row(t, _p(blocks[r * rs:]), _p(out[r]), ne0)
    return out


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.empty(row_size(Q8_0, x.size), dtype=np.uint8)
    lib().orc_quantize_row_q8_0(_p(x), _p(y), x.size)
    return y


def quantize_q8_K(x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.empty(row_size(Q8_K, x.size), dtype=np.uint8)
    lib().orc_quantize_row_q8_K(_p(x), _p(y), x.size)
    return y


def vec_dot(t, k, wrow, xq):
    return lib().orc_vec_dot(t, k, _p(np.ascontiguousarray(wrow)), _p(np.ascontiguousarray(xq)))


def mul_mat_ggml(t, W, N, K, x, nthreads=None):
    """W: uint8 GGUF bytes of N rows; x f32 [M, K] -> y f32 [M, N]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    lib().orc_mul_mat_ggml(t, _p(W), N, K, _p(x), K, M, _p(y), nthreads or default_threads())
    return y


def mul_mat_f64(t, W, N, K, x, nthreads=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    lib().orc_mul_mat_f64(t, _p(W), N, K, _p(x), K, M, _p(y), nthreads or default_threads())
    return y


# ---- flash attention ----
def make_tensor(arr, ggml_type, ne=None, nb=None):
    """Wrap a numpy array (kept alive by the caller) as an orc_tensor.

    Default ne/nb: the numpy array's axes reversed (ggml ne[0] = last axis)."""
    t = OrcTensor()
    t.data = arr.ctypes.data if arr is not None else None
    t.type = ggml_type
    if ne is None:
        shp = list(arr.shape)[::-1] + [1] * (4 - arr.ndim)
        st = list(arr.strides)[::-1] + [0] * (4 - arr.ndim)
        ne = shp
        nb = st
        for i in range(arr.ndim, 4):
            nb[i] = nb[i - 1] * ne[i - 1]
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t


def flash_attn_ext(q, k, v, mask, scale, flavour="ggml", nthreads=None, q_view=None):
    """q f32 [B, Hq, nq, D] (numpy, any strides), k/v f16 (as uint16 bits or
    float16) [Bk, Hkv, nkv, D], mask f16 [M3, M2, nq', nkv'] or None.

    Returns out [B, nq, Hq, D] (ggml's [D, Hq, nq, B]); float32 for the ggml
    flavour, float64 for "f64"."""
    k16 = k.view(np.uint16) if k.dtype == np.float16 else k
    v16 = v.view(np.uint16) if v.dtype == np.float16 else v
    tq = make_tensor(q, F32) if q_view is None else q_view
    tk = make_tensor(k16, F16)
    tv = make_tensor(v16, F16)
    m16 = None
    if mask is not None:
        m16 = mask.view(np.uint16) if mask.dtype == np.float16 else mask
        tm = make_tensor(m16, F16)
    else:
        tm = OrcTensor()
    B, Hq, nq, D = tq.ne[3], tq.ne[2], tq.ne[1], tq.ne[0]
    nt = nthreads or default_threads()
    if flavour == "ggml":
        out = np.empty((B, nq, Hq, D), dtype=np.float32)
        lib().orc_flash_attn_ext_ggml(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv),
                                      ctypes.byref(tm) if mask is not None else None, scale, _p(out), nt)
    else:
        out = np.empty((B, nq, Hq, D), dtype=np.float64)
        lib().orc_flash_attn_ext_f64(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv),
                                     ctypes.byref(tm) if mask is not None else None, scale, _p(out), nt)
    return out


# ---- glue ----
def rms_norm_mul(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = x.size // n
    y = np.empty_like(x)
    wp = _p(np.ascontiguousarray(w, dtype=np.float32)) if w is not None else None
    lib().orc_rms_norm_mul(_p(x), wp, _p(y), n, rows, eps)
    return y


def layer_norm(x, eps):
    """GGML_OP_NORM over the last axis (oracle.c orc_layer_norm)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_layer_norm(_p(x), _p(y), n, x.size // n, eps)
    return y


def rope_neox(x, positions, n_dims, freq_base):
    """x f32 [tokens, heads, head_dim]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H, D = x.shape
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    y = np.empty_like(x)
    lib().orc_rope_neox(_p(x), _p(y), D, n_dims, H, T, _p(pos), freq_base)
    return y


def swiglu(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1] // 2
    rows = x.size // (2 * n)
    y = np.empty(x.shape[:-1] + (n,), dtype=np.float32)
    lib().orc_swiglu(_p(x), _p(y), n, rows)
    return y
