"""ctypes binding of libmm_lm.so (include/mm_lm.h): the Qwen3-shape LM whose
batched CFG decode step runs, as a ggml graph, on the MI355X ggml backend."""
import ctypes
import pathlib

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libmm_lm.so"


class LmConfig(ctypes.Structure):
    _fields_ = [("n_layers", ctypes.c_int), ("hidden", ctypes.c_int), ("n_heads", ctypes.c_int),
                ("n_kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("ffn", ctypes.c_int),
                ("vocab", ctypes.c_int), ("max_seq", ctypes.c_int), ("n_sets", ctypes.c_int),
                ("wtype", ctypes.c_int), ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
                ("bump_type", ctypes.c_int)]


# Qwen3-8B shape of the decode benchmark (36 layers, vocab 151936, Q8_0)
QWEN3_8B = dict(n_layers=36, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=12288, vocab=151936,
                max_seq=4608, n_sets=2, wtype=8, rms_eps=1e-6, rope_theta=1e6)

_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i32, i64, u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64
        L.mm_lm_create.argtypes = [ctypes.POINTER(LmConfig), i32, u64]
        L.mm_lm_create.restype = vp
        L.mm_lm_create_on_backend.argtypes = [ctypes.POINTER(LmConfig), vp, u64]
        L.mm_lm_create_on_backend.restype = vp
        L.mm_lm_error.restype = ctypes.c_char_p
        L.mm_lm_free.argtypes = [vp]
        L.mm_lm_fill_kv.argtypes = [vp, i32, i32, u64]
        L.mm_lm_set_pos.argtypes = [vp, i32, i32]
        L.mm_lm_get_pos.argtypes = [vp, i32]
        L.mm_lm_decode.argtypes = [vp, vp, vp, i32, vp, vp]
        L.mm_lm_decode_device.argtypes = [vp, vp, vp, i32]
        L.mm_lm_tensor_nbytes.argtypes = [vp, ctypes.c_char_p]
        L.mm_lm_tensor_nbytes.restype = i64
        L.mm_lm_get_tensor.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_size_t]
        L.mm_lm_tensor_type.argtypes = [vp, ctypes.c_char_p]
        L.mm_lm_set_tensor.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_size_t]
        L.mm_lm_graph_nodes.argtypes = [vp]
        L.mm_lm_graph_stats.argtypes = [vp, ctypes.POINTER(i64), ctypes.POINTER(i64)]
        L.mm_lm_gpu_ms.restype = ctypes.c_double
        L.mm_lm_gpu_ms.argtypes = [vp, ctypes.c_int]
        _lib = L
    return _lib


class LmError(RuntimeError):
    pass


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


class Lm:
    def __init__(self, seed=1005, device=0, backend=None, **cfg):
        """backend: an existing MI355X ggml backend handle to share (e.g.
        OpGraph.backend; not freed by the LM), else one is created on device."""
        L = load()
        self.cfg = LmConfig(**cfg)
        if backend is not None:
            self.h = L.mm_lm_create_on_backend(ctypes.byref(self.cfg), backend, seed)
        else:
            self.h = L.mm_lm_create(ctypes.byref(self.cfg), device, seed)
        if not self.h:
            raise LmError(L.mm_lm_error().decode())

    def close(self):
        if self.h:
            load().mm_lm_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _check(self, rc):
        if rc != 0:
            raise LmError(load().mm_lm_error().decode())

    def fill_kv(self, s, n_pos, seed):
        self._check(load().mm_lm_fill_kv(self.h, s, n_pos, seed))

    def set_pos(self, s, pos):
        self._check(load().mm_lm_set_pos(self.h, s, pos))

    def pos(self, s):
        return load().mm_lm_get_pos(self.h, s)

    def decode(self, embeds, sets, want_logits=True, want_hidden=True):
        embeds = np.ascontiguousarray(embeds, np.float32)
        sets = np.ascontiguousarray(sets, np.int32)
        N = len(sets)
        logits = np.empty((N, self.cfg.vocab), np.float32) if want_logits else None
        hidden = np.empty((N, self.cfg.hidden), np.float32) if want_hidden else None
        self._check(load().mm_lm_decode(self.h, _p(embeds), _p(sets), N, _p(logits) if want_logits else None,
                                        _p(hidden) if want_hidden else None))
        return logits, hidden

    def decode_device(self, embeds, sets):
        embeds = np.ascontiguousarray(embeds, np.float32)
        sets = np.ascontiguousarray(sets, np.int32)
        self._check(load().mm_lm_decode_device(self.h, _p(embeds), _p(sets), len(sets)))

    def get(self, name, dtype=np.uint8):
        n = load().mm_lm_tensor_nbytes(self.h, name.encode())
        if n < 0:
            raise LmError(f"no tensor {name}")
        out = np.empty(n, np.uint8)
        self._check(load().mm_lm_get_tensor(self.h, name.encode(), _p(out), n))
        return out.view(dtype)

    def type_of(self, name):
        """GGML type of a weight or cache tensor; None if there is none."""
        t = load().mm_lm_tensor_type(self.h, name.encode())
        return None if t < 0 else t

    def has(self, name):
        return self.type_of(name) is not None

    def set(self, name, data):
        data = np.ascontiguousarray(data).view(np.uint8)
        self._check(load().mm_lm_set_tensor(self.h, name.encode(), _p(data), data.size))

    def graph_nodes(self):
        return load().mm_lm_graph_nodes(self.h)

    def gpu_ms(self, reset=False):
        """Mean GPU time per decode graph (ms) since the last reset."""
        return load().mm_lm_gpu_ms(self.h, 1 if reset else 0)

    def graph_stats(self):
        r, e = ctypes.c_int64(), ctypes.c_int64()
        load().mm_lm_graph_stats(self.h, ctypes.byref(r), ctypes.byref(e))
        return r.value, e.value
