"""ctypes view of the restated ggml API (libggml-base.so) for host-side tests."""
import ctypes
import pathlib

LIB = pathlib.Path(__file__).resolve().parent.parent / "minimaxmusic.cpp_amd" / "lib" / "libggml-base.so"
GGML_MAX_NAME = 128


class Tensor(ctypes.Structure):
    pass


Tensor._fields_ = [
    ("type", ctypes.c_int), ("buffer", ctypes.c_void_p), ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
    ("op", ctypes.c_int), ("op_params", ctypes.c_int32 * 16), ("flags", ctypes.c_int32),
    ("src", ctypes.POINTER(Tensor) * 10), ("view_src", ctypes.POINTER(Tensor)), ("view_offs", ctypes.c_size_t),
    ("data", ctypes.c_void_p), ("name", ctypes.c_char * GGML_MAX_NAME), ("extra", ctypes.c_void_p),
    ("padding", ctypes.c_char * 8),
]


class InitParams(ctypes.Structure):
    _fields_ = [("mem_size", ctypes.c_size_t), ("mem_buffer", ctypes.c_void_p), ("no_alloc", ctypes.c_bool)]


T = ctypes.POINTER(Tensor)


def load():
    L = ctypes.CDLL(str(LIB), mode=ctypes.RTLD_GLOBAL)
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    sig = {
        "ggml_init": (vp, [InitParams]), "ggml_free": (None, [vp]), "ggml_reset": (None, [vp]),
        "ggml_tensor_overhead": (sz, []), "ggml_graph_overhead_custom": (sz, [sz, ctypes.c_bool]),
        "ggml_new_tensor_1d": (T, [vp, i32, i64]), "ggml_new_tensor_2d": (T, [vp, i32, i64, i64]),
        "ggml_new_tensor_3d": (T, [vp, i32, i64, i64, i64]),
        "ggml_new_tensor_4d": (T, [vp, i32, i64, i64, i64, i64]),
        "ggml_view_2d": (T, [vp, T, i64, i64, sz, sz]), "ggml_view_4d": (T, [vp, T, i64, i64, i64, i64, sz, sz, sz, sz]),
        "ggml_reshape_3d": (T, [vp, T, i64, i64, i64]), "ggml_reshape_4d": (T, [vp, T, i64, i64, i64, i64]),
        "ggml_permute": (T, [vp, T, i32, i32, i32, i32]), "ggml_cont": (T, [vp, T]), "ggml_cast": (T, [vp, T, i32]),
        "ggml_mul_mat": (T, [vp, T, T]), "ggml_add": (T, [vp, T, T]), "ggml_mul": (T, [vp, T, T]),
        "ggml_rms_norm": (T, [vp, T, f32]), "ggml_swiglu": (T, [vp, T]), "ggml_set_rows": (T, [vp, T, T, T]),
        "ggml_get_rows": (T, [vp, T, T]),
        "ggml_rope_ext": (T, [vp, T, T, T, i32, i32, i32, f32, f32, f32, f32, f32, f32]),
        "ggml_flash_attn_ext": (T, [vp, T, T, T, T, f32, f32, f32]), "ggml_flash_attn_ext_set_prec": (None, [T, i32]),
        "ggml_new_graph_custom": (vp, [vp, sz, ctypes.c_bool]), "ggml_build_forward_expand": (None, [vp, T]),
        "ggml_graph_n_nodes": (i32, [vp]), "ggml_graph_node": (T, [vp, i32]), "ggml_graph_n_leafs": (i32, [vp]),
        "ggml_nbytes": (sz, [T]), "ggml_row_size": (sz, [i32, i64]), "ggml_is_contiguous": (ctypes.c_bool, [T]),
        "ggml_op_name": (ctypes.c_char_p, [i32]), "ggml_set_name": (T, [T, ctypes.c_char_p]),
        "ggml_fp32_to_fp16": (ctypes.c_uint16, [f32]), "ggml_fp16_to_fp32": (f32, [ctypes.c_uint16]),
    }
    for n, (r, a) in sig.items():
        fn = getattr(L, n)
        fn.restype = r
        fn.argtypes = a
    return L
