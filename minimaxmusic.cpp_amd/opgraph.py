"""Single-op ggml graphs run through the MI355X ggml backend (ctypes).

The reference hands every op to a ggml backend inside a graph
(ggml_backend_sched_graph_compute, src/qwen3-lm.h:620, src/dit.h:385, or
ggml_backend_graph_compute, src/static-graph.h:58).  This module builds graphs
of FLASH_ATTN_EXT / MUL_MAT nodes and of the DiT block's glue ops with the restated ggml API
(libggml-base.so), allocates them in the backend's device buffer, uploads
inputs with ggml_backend_tensor_set (quantized weights as GGUF blocks: the
buffer repacks them) and runs ggml_backend_graph_compute on the MI355X backend
(libggml-mi355x.so): the eager first call, then HIP-graph capture and replays.
There is no CPU path: the backend library must load and find a GPU.
"""
import ctypes
import pathlib

import numpy as np

LIBDIR = pathlib.Path(__file__).resolve().parent / "lib"
GGML_MAX_NAME = 128
F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 8, 12, 13, 14, 30
PREC_F32 = 10
ROPE_NEOX = 2


class Tensor(ctypes.Structure):
    pass


Tensor._fields_ = [
    ("type", ctypes.c_int), ("buffer", ctypes.c_void_p), ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
    ("op", ctypes.c_int), ("op_params", ctypes.c_int32 * 16), ("flags", ctypes.c_int32),
    ("src", ctypes.POINTER(Tensor) * 10), ("view_src", ctypes.POINTER(Tensor)), ("view_offs", ctypes.c_size_t),
    ("data", ctypes.c_void_p), ("name", ctypes.c_char * GGML_MAX_NAME), ("extra", ctypes.c_void_p),
    ("padding", ctypes.c_char * 8),
]


class _InitParams(ctypes.Structure):
    _fields_ = [("mem_size", ctypes.c_size_t), ("mem_buffer", ctypes.c_void_p), ("no_alloc", ctypes.c_bool)]


_T = ctypes.POINTER(Tensor)
_libs = {}


def _load():
    if _libs:
        return _libs["base"], _libs["mi"]
    vp, i64, i32, f32, sz, b = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_bool
    base = ctypes.CDLL(str(LIBDIR / "libggml-base.so"), mode=ctypes.RTLD_GLOBAL)
    mi = ctypes.CDLL(str(LIBDIR / "libggml-mi355x.so"), mode=ctypes.RTLD_GLOBAL)
    sig = {
        "ggml_init": (vp, [_InitParams]), "ggml_free": (None, [vp]),
        "ggml_tensor_overhead": (sz, []), "ggml_graph_overhead_custom": (sz, [sz, b]),
        "ggml_new_tensor_4d": (_T, [vp, i32, i64, i64, i64, i64]),
        "ggml_mul_mat": (_T, [vp, _T, _T]),
        "ggml_add": (_T, [vp, _T, _T]), "ggml_mul": (_T, [vp, _T, _T]),
        "ggml_norm": (_T, [vp, _T, f32]), "ggml_scale": (_T, [vp, _T, f32]),
        "ggml_clamp": (_T, [vp, _T, f32, f32]), "ggml_concat": (_T, [vp, _T, _T, i32]),
        "ggml_rope_ext": (_T, [vp, _T, _T, _T, i32, i32, i32, f32, f32, f32, f32, f32, f32]),
        "ggml_permute": (_T, [vp, _T, i32, i32, i32, i32]),
        "ggml_reshape_3d": (_T, [vp, _T, i64, i64, i64]), "ggml_reshape_4d": (_T, [vp, _T, i64, i64, i64, i64]),
        "ggml_view_3d": (_T, [vp, _T, i64, i64, i64, sz, sz, sz]),
        "ggml_cast": (_T, [vp, _T, i32]), "ggml_cont": (_T, [vp, _T]),
        "ggml_swiglu_split": (_T, [vp, _T, _T]),
        "ggml_rms_norm": (_T, [vp, _T, f32]), "ggml_transpose": (_T, [vp, _T]),
        "ggml_soft_max": (_T, [vp, _T]), "ggml_diag_mask_inf": (_T, [vp, _T, i32]),
        "ggml_sub": (_T, [vp, _T, _T]), "ggml_scale_bias": (_T, [vp, _T, f32, f32]),
        "ggml_argsort_top_k": (_T, [vp, _T, i32]), "ggml_cumsum": (_T, [vp, _T]), "ggml_sum": (_T, [vp, _T]),
        "ggml_step": (_T, [vp, _T]), "ggml_get_rows": (_T, [vp, _T, _T]),
        "ggml_reshape_1d": (_T, [vp, _T, i64]), "ggml_reshape_2d": (_T, [vp, _T, i64, i64]),
        "ggml_view_1d": (_T, [vp, _T, i64, sz]),
        "ggml_flash_attn_ext": (_T, [vp, _T, _T, _T, _T, f32, f32, f32]),
        "ggml_flash_attn_ext_set_prec": (None, [_T, i32]),
        "ggml_new_graph_custom": (vp, [vp, sz, b]), "ggml_build_forward_expand": (None, [vp, _T]),
        "ggml_nbytes": (sz, [_T]),
        "ggml_backend_alloc_ctx_tensors": (vp, [vp, vp]), "ggml_backend_buffer_free": (None, [vp]),
        "ggml_backend_tensor_set": (None, [_T, vp, sz, sz]), "ggml_backend_tensor_get": (None, [_T, vp, sz, sz]),
        "ggml_backend_graph_compute": (i32, [vp, vp]), "ggml_backend_synchronize": (None, [vp]),
        "ggml_backend_free": (None, [vp]),
    }
    for n, (r, a) in sig.items():
        fn = getattr(base, n)
        fn.restype, fn.argtypes = r, a
    misig = {
        "ggml_backend_mi355x_init": (vp, [i32]),
        "ggml_backend_mi355x_gpu_time": (None, [vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(i64), i32]),
        "ggml_backend_mi355x_graph_stats": (None, [vp, ctypes.POINTER(i64), ctypes.POINTER(i64)]),
        "ggml_backend_mi355x_graph_cache_info": (None, [vp, ctypes.POINTER(i64), ctypes.POINTER(i64),
                                                        ctypes.POINTER(i64)]),
        "ggml_backend_mi355x_f16_weight_bytes": (ctypes.c_size_t, []),
    }
    for n, (r, a) in misig.items():
        fn = getattr(mi, n)
        fn.restype, fn.argtypes = r, a
    _libs["base"], _libs["mi"] = base, mi
    return base, mi


class OpGraph:
    """A ggml context of graph tensors on the MI355X backend.  Create the
    tensors and ops, call build(outputs), upload inputs with set(), then
    compute() runs the graph through ggml_backend_graph_compute."""

    def __init__(self, n_tensors=256, device=0, backend=None):
        """backend: an MI355X backend handle to share with other graphs (not
        freed by close()), else a new one on `device`."""
        self.G, self.MI = _load()
        mem = n_tensors * self.G.ggml_tensor_overhead() + self.G.ggml_graph_overhead_custom(n_tensors, False)
        self.ctx = self.G.ggml_init(_InitParams(mem, None, True))
        if not self.ctx:
            raise RuntimeError("ggml_init failed")
        self.owns_backend = backend is None
        self.backend = self.MI.ggml_backend_mi355x_init(device) if backend is None else backend
        if not self.backend:
            raise RuntimeError("MI355X ggml backend: no device")
        self.n_tensors = n_tensors
        self.buf = None
        self.graph = None

    def tensor(self, type_, ne):
        ne = list(ne) + [1] * (4 - len(ne))
        return self.G.ggml_new_tensor_4d(self.ctx, type_, *ne)

    def flash_attn(self, q, k, v, mask, scale):
        t = self.G.ggml_flash_attn_ext(self.ctx, q, k, v, mask, scale, 0.0, 0.0)
        self.G.ggml_flash_attn_ext_set_prec(t, PREC_F32)
        return t

    def mul_mat(self, w, x):
        return self.G.ggml_mul_mat(self.ctx, w, x)

    # the DiT block's other ops (src/dit.h:161-247, :255-268)
    def add(self, a, b):
        return self.G.ggml_add(self.ctx, a, b)

    def mul(self, a, b):
        return self.G.ggml_mul(self.ctx, a, b)

    def norm(self, a, eps):
        return self.G.ggml_norm(self.ctx, a, eps)

    def scale(self, a, s):
        return self.G.ggml_scale(self.ctx, a, s)

    def clamp(self, a, lo, hi):
        return self.G.ggml_clamp(self.ctx, a, lo, hi)

    def concat(self, a, b, dim):
        return self.G.ggml_concat(self.ctx, a, b, dim)

    def rope_neox(self, a, pos, n_dims, freq_base):
        return self.G.ggml_rope_ext(self.ctx, a, pos, None, n_dims, ROPE_NEOX, 0, freq_base, 1.0, 0.0, 1.0, 0.0, 0.0)

    def permute(self, a, *axes):
        return self.G.ggml_permute(self.ctx, a, *axes)

    def reshape(self, a, ne):
        if len(ne) == 3:
            return self.G.ggml_reshape_3d(self.ctx, a, *ne)
        return self.G.ggml_reshape_4d(self.ctx, a, *ne)

    def view_3d(self, a, ne, nb1, nb2, offset):
        return self.G.ggml_view_3d(self.ctx, a, ne[0], ne[1], ne[2], nb1, nb2, offset)

    def cast(self, a, type_):
        return self.G.ggml_cast(self.ctx, a, type_)

    def cont(self, a):
        return self.G.ggml_cont(self.ctx, a)

    def swiglu_split(self, gate, value):
        return self.G.ggml_swiglu_split(self.ctx, gate, value)

    # the depth decoder's layer (src/depth-decoder.h:192-236)
    def rms_norm(self, a, eps):
        return self.G.ggml_rms_norm(self.ctx, a, eps)

    def transpose(self, a):
        return self.G.ggml_transpose(self.ctx, a)

    def soft_max(self, a):
        return self.G.ggml_soft_max(self.ctx, a)

    def diag_mask_inf(self, a, n_past):
        return self.G.ggml_diag_mask_inf(self.ctx, a, n_past)

    # the depth decoder's in-graph sampler (src/depth-decoder.h:331-361)
    def sub(self, a, b):
        return self.G.ggml_sub(self.ctx, a, b)

    def scale_bias(self, a, s, b):
        return self.G.ggml_scale_bias(self.ctx, a, s, b)

    def argsort_top_k(self, a, k):
        return self.G.ggml_argsort_top_k(self.ctx, a, k)

    def cumsum(self, a):
        return self.G.ggml_cumsum(self.ctx, a)

    def sum(self, a):
        return self.G.ggml_sum(self.ctx, a)

    def step(self, a):
        return self.G.ggml_step(self.ctx, a)

    def get_rows(self, a, idx):
        return self.G.ggml_get_rows(self.ctx, a, idx)

    def reshape_1d(self, a, n0):
        return self.G.ggml_reshape_1d(self.ctx, a, n0)

    def reshape_2d(self, a, n0, n1):
        return self.G.ggml_reshape_2d(self.ctx, a, n0, n1)

    def view_1d(self, a, n0, offset):
        return self.G.ggml_view_1d(self.ctx, a, n0, offset)

    def build(self, outputs):
        self.graph = self.G.ggml_new_graph_custom(self.ctx, self.n_tensors, False)
        for t in outputs:
            self.G.ggml_build_forward_expand(self.graph, t)
        self.buf = self.G.ggml_backend_alloc_ctx_tensors(self.ctx, self.backend)
        if not self.buf:
            raise RuntimeError("ggml_backend_alloc_ctx_tensors failed")

    def set(self, t, arr):
        a = np.ascontiguousarray(arr)
        n = self.G.ggml_nbytes(t)
        if a.nbytes != n:
            raise ValueError(f"tensor_set: {a.nbytes} bytes for a {n}-byte tensor")
        self.G.ggml_backend_tensor_set(t, a.ctypes.data_as(ctypes.c_void_p), 0, n)

    def get(self, t, dtype=np.float32):
        n = self.G.ggml_nbytes(t)
        out = np.empty(n // np.dtype(dtype).itemsize, dtype=dtype)
        self.G.ggml_backend_tensor_get(t, out.ctypes.data_as(ctypes.c_void_p), 0, n)
        return out

    def compute(self):
        rc = self.G.ggml_backend_graph_compute(self.backend, self.graph)
        if rc != 0:
            raise RuntimeError(f"ggml_backend_graph_compute: status {rc}")

    def synchronize(self):
        self.G.ggml_backend_synchronize(self.backend)

    def gpu_time(self, reset=False):
        """(total GPU ms, graph_compute calls) since the last reset: HIP
        events on the backend stream around each graph_compute."""
        ms, n = ctypes.c_double(0.0), ctypes.c_int64(0)
        self.MI.ggml_backend_mi355x_gpu_time(self.backend, ctypes.byref(ms), ctypes.byref(n), 1 if reset else 0)
        return ms.value, n.value

    def graph_stats(self):
        r, e = ctypes.c_int64(0), ctypes.c_int64(0)
        self.MI.ggml_backend_mi355x_graph_stats(self.backend, ctypes.byref(r), ctypes.byref(e))
        return r.value, e.value

    def f16_weight_bytes(self):
        """Bytes of f16 weight copies the backend holds (process-wide)."""
        return int(self.MI.ggml_backend_mi355x_f16_weight_bytes())

    def graph_cache_info(self):
        """(graphs kept by the backend, of which captured, captures so far)."""
        a, b, c = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
        self.MI.ggml_backend_mi355x_graph_cache_info(self.backend, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
        return a.value, b.value, c.value

    def close(self):
        # the backend first: it waits for its stream and drops the captured
        # HIP graphs that point into the buffer, then the buffer goes
        if self.backend:
            if self.owns_backend:
                self.G.ggml_backend_free(self.backend)
            else:
                self.G.ggml_backend_synchronize(self.backend)
            self.backend = None
        if self.buf:
            self.G.ggml_backend_buffer_free(self.buf)
            self.buf = None
        if self.ctx:
            self.G.ggml_free(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
