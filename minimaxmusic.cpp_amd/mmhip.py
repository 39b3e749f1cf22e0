"""Python host mirror of the MI355X kernel C-ABI (include/mmhip.h).

Loads lib/libmmhip.so with ctypes and exposes the two ggml ops of the hot path
with the reference's argument meaning:

* ``mul_mat(W, x)``: GGML_OP_MUL_MAT with a quantized src0 (``W``, a
  :class:`QuantWeight` in the device row-grouped layout) and an f32 src1
  (``x``, ``[M, K]``): ``y[M, N] = x @ deq(W).T`` - ggml's
  ``dst[n, m] = sum_k W[k, n] x[k, m]`` in ggml's ``ne`` order
  (src/qwen3-enc.h:67-69).
* ``flash_attn_ext(q, k, v, mask, scale)``: GGML_OP_FLASH_ATTN_EXT with ggml's
  operand layouts given as torch views (src/qwen3-lm.h:816-821,
  src/dit.h:221-222).  Errors raise :class:`MmhipError` carrying the C-ABI
  status, as the ggml backend would return a ``GGML_STATUS_*``.

torch is used only to own device memory and streams.  There is no fallback:
if the library is missing or no GPU is visible, calls raise.
"""
import ctypes
import pathlib

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libmmhip.so"

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 8, 12, 13, 14, 15
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_WORKSPACE = 0, -1, -2, -3, -4


class MmhipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"mmhip error {code}: {msg}")
        self.code = code


class MmhipView(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_int64 * 4)]


class HeadRowsArgs(ctypes.Structure):
    """mmhip_head_rows_args (include/mmhip.h)."""
    _fields_ = [("src", ctypes.c_void_p), ("src_nb_h", ctypes.c_int64), ("src_nb_t", ctypes.c_int64),
                ("D", ctypes.c_int), ("H", ctypes.c_int), ("T", ctypes.c_int), ("norm", ctypes.c_int),
                ("norm_w", ctypes.c_void_p), ("eps", ctypes.c_float), ("pos", ctypes.c_void_p),
                ("theta_scale", ctypes.c_float), ("dst", ctypes.c_void_p), ("dst_type", ctypes.c_int),
                ("ids", ctypes.c_void_p), ("ids_type", ctypes.c_int), ("ids_nb1", ctypes.c_int64),
                ("ids_nb2", ctypes.c_int64), ("ids_ne1", ctypes.c_int64), ("ids_ne2", ctypes.c_int64),
                ("dst_nb1", ctypes.c_int64), ("dst_nb2", ctypes.c_int64), ("dst_nb3", ctypes.c_int64)]


# Every symbol include/mmhip.h declares, with (restype, argtypes).
_vp, _i64, _i32, _f32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
_VP = ctypes.POINTER(MmhipView)
SIGNATURES = {
    "mmhip_last_error": (ctypes.c_char_p, []),
    "mmhip_version": (_i32, []),
    "mmhip_repack_rows": (_i32, [_i32, _vp, _vp, _i64, _i64, _vp]),
    "mmhip_unpack_rows": (_i32, [_i32, _vp, _vp, _i64, _i64, _vp]),
    "mmhip_dequantize_rows": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _vp]),
    "mmhip_mul_mat_workspace": (_sz, [_i32, _i64, _i64, _i64]),
    "mmhip_mul_mat": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _sz, _vp]),
    "mmhip_mul_mat_bf16": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp]),
    "mmhip_mul_mat_bf16_dec_supported": (_i32, [_i64, _i64, _i64, _i32]),
    "mmhip_mul_mat_bf16_dec": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _f32, _vp, _i64, _i32, _vp, _i64,
                                      _vp]),
    "mmhip_mul_mat_bias_add": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp,
                                      _sz, _vp]),
    "mmhip_mul_mat_bias_add_h": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp]),
    "mmhip_mul_mat_bias_swiglu": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i32, _vp, _vp, _vp, _sz,
                                         _vp]),
    "mmhip_mul_mat_bias_swiglu_h": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _vp, _vp]),
    "mmhip_mul_mat_h_workspace": (_sz, [_i32, _i64, _i64, _i64]),
    "mmhip_weights_f16_bytes": (_sz, [_i64, _i64]),
    "mmhip_weights_to_f16": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _vp]),
    "mmhip_register_weights_f16": (_i32, [_vp, _i64, _i64, _vp]),
    "mmhip_unregister_weights_f16": (_i32, [_vp]),
    "mmhip_mul_mat_bias_add_hw": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _sz,
                                         _vp]),
    "mmhip_mul_mat_multi": (_i32, [_i32, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mmhip_mul_mat_multi_h": (_i32, [_i32, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _vp]),
    "mmhip_act_bytes": (_sz, [_i32, _i64, _i64]),
    "mmhip_quantize_act": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _vp]),
    "mmhip_mul_mat_q": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "mmhip_mul_mat_q_add": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "mmhip_flash_attn_ext_head_supported": (_i32, [_VP, _VP, _VP]),
    "mmhip_flash_attn_ext_head": (_i32, [_VP, _VP, _VP, _VP, _f32, _vp, _vp, _sz, _i32, _vp, _vp, _vp]),
    "mmhip_rms_norm_mul_mat_supported": (_i32, [_i32, _i64, _i64, _i64]),
    "mmhip_rms_norm_mul_mat": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _f32, _vp, _vp, _i64, _vp,
                                      _i64, _vp]),
    "mmhip_swiglu_mul_mat_supported": (_i32, [_i32, _i64, _i64, _i64]),
    "mmhip_swiglu_mul_mat": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp,
                                    _i64, _vp]),
    "mmhip_rms_norm_mul_mat_glu_supported": (_i32, [_i32, _i64, _i64, _i64]),
    "mmhip_rms_norm_mul_mat_glu": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _f32, _i32, _vp, _vp,
                                          _vp]),
    "mmhip_flash_attn_workspace": (_sz, [_VP, _VP, _VP]),
    "mmhip_flash_attn_ext": (_i32, [_VP, _VP, _VP, _VP, _f32, _vp, _vp, _sz, _vp]),
    "mmhip_flash_attn_noalloc_max_workspace": (_sz, []),
    "mmhip_flash_attn_ext_noalloc": (_i32, [_VP, _VP, _VP, _VP, _f32, _vp, _vp]),
    "mmhip_flash_attn_ext_q": (_i32, [_VP, _VP, _VP, _VP, _f32, _vp, _vp, _sz, _i32, _vp, _vp]),
    "mmhip_binary": (_i32, [_i32, _VP, _VP, _vp, _vp]),
    "mmhip_rms_norm": (_i32, [_VP, _VP, _f32, _vp, _vp]),
    "mmhip_rms_norm_quant": (_i32, [_VP, _VP, _f32, _vp, _i32, _vp, _vp]),
    "mmhip_head_rows": (_i32, [ctypes.c_void_p, _vp]),
    "mmhip_head_rows_n": (_i32, [ctypes.c_void_p, _i32, _vp]),
    "mmhip_swiglu_quant": (_i32, [_VP, _VP, _i32, _vp, _i32, _vp, _vp]),
    "mmhip_rope_neox": (_i32, [_VP, _vp, _i32, _f32, _vp, _vp]),
    "mmhip_rope_neox_f16": (_i32, [_VP, _vp, _i32, _f32, _VP, _vp]),
    "mmhip_cpy": (_i32, [_VP, _i32, _VP, _i32, _vp]),
    "mmhip_get_rows": (_i32, [_i32, _VP, _VP, _vp, _vp]),
    "mmhip_set_rows": (_i32, [_VP, _VP, _i32, _VP, _i32, _vp]),
    "mmhip_swiglu": (_i32, [_VP, _VP, _i32, _vp, _vp]),
    "mmhip_scale": (_i32, [_VP, _f32, _f32, _vp, _vp]),
    "mmhip_norm": (_i32, [_VP, _f32, _vp, _vp]),
    "mmhip_norm_affine": (_i32, [_VP, _f32, _vp, _vp, _vp, _vp]),
    "mmhip_norm_affine_h": (_i32, [_VP, _f32, _vp, _vp, _vp, _vp, _vp]),
    "mmhip_concat": (_i32, [_VP, _VP, _i32, _vp, _vp]),
    "mmhip_mul_mat_f32": (_i32, [_VP, _VP, _vp, _vp]),
    "mmhip_diag_mask_inf": (_i32, [_VP, _i32, _vp, _vp]),
    "mmhip_soft_max": (_i32, [_VP, _vp, _vp]),
    "mmhip_small_attn": (_i32, [_VP, _VP, _VP, _f32, _f32, _i32, _vp, _vp]),
    "mmhip_small_attn_q": (_i32, [_VP, _VP, _VP, _f32, _f32, _i32, _vp, _i32, _vp, _vp]),
    "mmhip_argsort_desc": (_i32, [_VP, _vp, _vp]),
    "mmhip_cumsum": (_i32, [_VP, _vp, _vp]),
    "mmhip_sum": (_i32, [_VP, _vp, _vp]),
    "mmhip_step": (_i32, [_VP, _vp, _vp]),
    "mmhip_cast_i32": (_i32, [_VP, _vp, _vp]),
    "mmhip_cast_f32_of_i32": (_i32, [_VP, _vp, _vp]),
    "mmhip_clamp": (_i32, [_VP, _f32, _f32, _vp, _vp]),
    # include/mmhip_synth.h
    "mmhip_synth_gguf": (_i32, [_i32, _vp, _i64, ctypes.c_uint64, _vp]),
    "mmhip_synth_normal": (_i32, [_i32, _vp, _i64, ctypes.c_uint64, _f32, _f32, _vp]),
}

_lib = None


def load(path=None):
    """Load the kernel library (raises if it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path) if path else LIB_PATH
    if not p.exists():
        raise MmhipError(ERR_UNSUPPORTED, f"{p} is not built; run __graft_entry__.build()")
    L = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = L
    return L


def _check(rc):
    if rc != OK:
        raise MmhipError(rc, load().mmhip_last_error().decode())


def _torch():
    import torch

    if not torch.cuda.is_available():
        raise MmhipError(ERR_HIP, "no GPU visible")
    return torch


def _stream():
    return ctypes.c_void_p(_torch().cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def row_size(t, ne0):
    be, bb = BLOCK[t]
    return ne0 // be * bb


def view_of(t, ne=None, nb=None):
    """mmhip_view of a torch tensor; by default ggml order = torch dims reversed."""
    v = MmhipView()
    v.data = t.data_ptr()
    es = t.element_size()
    if ne is None:
        shp = list(t.shape)[::-1]
        st = [s * es for s in list(t.stride())[::-1]]
        while len(shp) < 4:
            st.append(st[-1] * shp[-1] if shp else es)
            shp.append(1)
        ne, nb = shp, st
    for i in range(4):
        v.ne[i] = int(ne[i])
        v.nb[i] = int(nb[i])
    return v


class QuantWeight:
    """A quantized weight [N rows x K] resident on the device in the row-grouped
    layout (same byte size as the GGUF rows)."""

    def __init__(self, qtype, data, N, K):
        self.qtype, self.data, self.N, self.K = qtype, data, N, K
        self.row_bytes = row_size(qtype, K)

    @classmethod
    def from_gguf(cls, qtype, gguf_bytes, N, K):
        """Upload GGUF blocks (host numpy uint8 or device uint8 tensor) and repack."""
        torch = _torch()
        src = gguf_bytes
        if not isinstance(src, torch.Tensor):
            src = torch.from_numpy(src.reshape(-1)).to("cuda")
        assert src.numel() == N * row_size(qtype, K)
        dst = torch.empty_like(src)
        _check(load().mmhip_repack_rows(qtype, _ptr(src), _ptr(dst), N, K, _stream()))
        return cls(qtype, dst, N, K)

    def to_gguf(self):
        torch = _torch()
        out = torch.empty_like(self.data)
        _check(load().mmhip_unpack_rows(self.qtype, _ptr(self.data), _ptr(out), self.N, self.K, _stream()))
        return out

    def dequantize(self):
        torch = _torch()
        out = torch.empty((self.N, self.K), dtype=torch.float32, device=self.data.device)
        _check(load().mmhip_dequantize_rows(self.qtype, _ptr(self.data), self.N, self.K, self.row_bytes, _ptr(out),
                                            _stream()))
        return out


def mul_mat(W, x, out=None, workspace=None):
    """y[M, N] = x[M, K] @ deq(W).T on the GPU (GGML_OP_MUL_MAT)."""
    torch = _torch()
    assert x.dtype == torch.float32 and x.dim() == 2 and x.shape[1] == W.K and x.stride(1) == 1
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, W.N), dtype=torch.float32, device=x.device)
    L = load()
    need = L.mmhip_mul_mat_workspace(W.qtype, W.N, W.K, M)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    wsp = _ptr(workspace) if need else None
    _check(L.mmhip_mul_mat(W.qtype, _ptr(W.data), W.N, W.K, W.row_bytes, _ptr(x), x.stride(0), M, _ptr(out),
                           out.stride(0), wsp, need, _stream()))
    return out


def mul_mat_bias_swiglu(W, x, bias=None, swapped=False, f32_out=True, f16_out=False, workspace=None):
    """silu(gate) * value over the two halves of (x @ deq(W).T + bias) in the
    GEMM's epilogue (value = first W.N / 2 rows, gate = the rest; swapped:
    the other way round).  x is f32 [M, K] or f16 [M, K] (then used as the
    GEMM's activation copy).  Returns (h f32 [M, F] or None, hh f16 or None)."""
    torch = _torch()
    assert x.dim() == 2 and x.shape[1] == W.K and x.stride(1) == 1 and W.N % 2 == 0
    M, F = x.shape[0], W.N // 2
    h = torch.empty((M, F), dtype=torch.float32, device=x.device) if f32_out else None
    hh = torch.empty((M, F), dtype=torch.float16, device=x.device) if f16_out else None
    L = load()
    bp = _ptr(bias) if bias is not None else None
    if x.dtype == torch.float16:
        assert x.is_contiguous()
        _check(L.mmhip_mul_mat_bias_swiglu_h(W.qtype, _ptr(W.data), W.N, W.K, W.row_bytes, _ptr(x), M, bp,
                                             int(swapped), _ptr(h) if h is not None else None,
                                             _ptr(hh) if hh is not None else None, _stream()))
        return h, hh
    assert x.dtype == torch.float32
    need = L.mmhip_mul_mat_workspace(W.qtype, W.N, W.K, M)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _check(L.mmhip_mul_mat_bias_swiglu(W.qtype, _ptr(W.data), W.N, W.K, W.row_bytes, _ptr(x), x.stride(0), M, bp,
                                       int(swapped), _ptr(h) if h is not None else None,
                                       _ptr(hh) if hh is not None else None, _ptr(workspace) if need else None, need,
                                       _stream()))
    return h, hh


def mul_mat_bias_add(W, x, bias=None, r=None, out=None, workspace=None):
    """y = x @ deq(W).T (+ bias) (+ r), the GEMM with its ADDs in the store."""
    torch = _torch()
    assert x.dtype == torch.float32 and x.dim() == 2 and x.shape[1] == W.K and x.stride(1) == 1
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, W.N), dtype=torch.float32, device=x.device)
    L = load()
    need = L.mmhip_mul_mat_workspace(W.qtype, W.N, W.K, M)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _check(L.mmhip_mul_mat_bias_add(W.qtype, _ptr(W.data), W.N, W.K, W.row_bytes, _ptr(x), x.stride(0), M,
                                    _ptr(bias) if bias is not None else None, _ptr(r) if r is not None else None,
                                    r.stride(0) if r is not None else 0, _ptr(out), out.stride(0),
                                    _ptr(workspace) if need else None, need, _stream()))
    return out


def quantize_act(qtype, x):
    torch = _torch()
    M, K = x.shape
    n = load().mmhip_act_bytes(qtype, K, M)
    if n == 0:
        raise MmhipError(ERR_UNSUPPORTED, f"no activation layout for type {qtype}, K={K}")
    buf = torch.empty(n, dtype=torch.uint8, device=x.device)
    _check(load().mmhip_quantize_act(qtype, _ptr(x), x.stride(0), K, M, _ptr(buf), _stream()))
    return buf


def flash_attn_ext(q, k, v, mask, scale, out=None, q_view=None, k_view=None, v_view=None, mask_view=None,
                   workspace=None):
    """GGML_OP_FLASH_ATTN_EXT.

    q f32 [B, Hq, nq, D], k/v f16 [Bk, Hkv, nkv, D], mask f16 [M3, M2, nq', nkv']
    or None (torch dims = ggml dims reversed; any strides, or explicit ggml
    views).  Returns f32 [B, nq, Hq, D] (ggml's [D, Hq, nq, B])."""
    torch = _torch()
    qv = q_view or view_of(q)
    kv = k_view or view_of(k)
    vv = v_view or view_of(v)
    mv = mask_view or (view_of(mask) if mask is not None else None)
    D, nq, Hq, B = qv.ne[0], qv.ne[1], qv.ne[2], qv.ne[3]
    if out is None:
        out = torch.empty((B, nq, Hq, D), dtype=torch.float32, device=q.device)
    L = load()
    need = L.mmhip_flash_attn_workspace(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv))
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _check(L.mmhip_flash_attn_ext(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                  ctypes.byref(mv) if mv is not None else None, scale, _ptr(out),
                                  _ptr(workspace) if need else None, need, _stream()))
    return out
