"""Host-side checks of the restated ggml API (graph building, views, shapes,
op parameters) that the MI355X backend consumes.  No GPU needed."""
import math

import numpy as np
import pytest

import ggml_ctypes as G

F32, F16, Q8_0, Q4_K, Q6_K, I32, I64 = 0, 1, 8, 12, 14, 26, 27


@pytest.fixture(scope="module")
def L():
    import __graft_entry__

    if not G.LIB.exists():
        __graft_entry__.build()
    return G.load()


@pytest.fixture
def ctx(L):
    c = L.ggml_init(G.InitParams(64 << 20, None, True))
    yield c
    L.ggml_free(c)


def test_row_sizes_and_fp16(L):
    assert L.ggml_row_size(Q8_0, 4096) == 4096 // 32 * 34
    assert L.ggml_row_size(Q4_K, 2048) == 8 * 144
    assert L.ggml_row_size(Q6_K, 4096) == 16 * 210
    x = np.random.default_rng(0).standard_normal(2000).astype(np.float32)
    got = np.array([L.ggml_fp32_to_fp16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))
    assert L.ggml_fp16_to_fp32(0x3C00) == 1.0


def test_tensor_layout_and_views(L, ctx):
    assert G.ctypes.sizeof(G.Tensor) == 400  # GGML_MAX_NAME = 128 (reference CMakeLists.txt:33-34)
    a = L.ggml_new_tensor_3d(ctx, F32, 128, 32, 2)
    t = a.contents
    assert list(t.ne) == [128, 32, 2, 1] and list(t.nb) == [4, 512, 512 * 32, 512 * 64]
    p = L.ggml_permute(ctx, a, 0, 2, 1, 3).contents
    assert list(p.ne) == [128, 2, 32, 1] and list(p.nb)[:3] == [4, 512 * 32, 512]
    assert not L.ggml_is_contiguous(L.ggml_permute(ctx, a, 0, 2, 1, 3))
    v = L.ggml_view_2d(ctx, a, 64, 32, 512, 256).contents
    assert v.view_offs == 256 and v.nb[1] == 512 and L.ggml_op_name(v.op) == b"VIEW"
    w = L.ggml_new_tensor_2d(ctx, Q8_0, 4096, 100)
    assert L.ggml_nbytes(w) == 100 * 4352


def test_decode_attention_block_graph(L, ctx):
    """The attention part of qw3lm_forward_batch (src/qwen3-lm.h:742-823) builds
    the expected node sequence with the expected shapes and op params."""
    H, D, Nh, Nkv, N, S, pad = 4096, 128, 32, 8, 2, 4096, 2304
    gf = L.ggml_new_graph_custom(ctx, 4096, False)
    x = L.ggml_new_tensor_2d(ctx, F32, H, N)
    wqkv = L.ggml_new_tensor_2d(ctx, Q8_0, H, Nh * D + 2 * Nkv * D)
    pos = L.ggml_new_tensor_1d(ctx, I32, N)
    rows = L.ggml_new_tensor_3d(ctx, I64, 1, 1, N)
    mask = L.ggml_new_tensor_4d(ctx, F16, pad, 1, 1, N)
    kc = L.ggml_new_tensor_4d(ctx, F16, D, S, Nkv, N)
    qkv = L.ggml_mul_mat(ctx, wqkv, x)
    assert list(qkv.contents.ne) == [Nh * D + 2 * Nkv * D, N, 1, 1]
    q = L.ggml_cont(ctx, L.ggml_view_2d(ctx, qkv, Nh * D, N, qkv.contents.nb[1], 0))
    k = L.ggml_cont(ctx, L.ggml_view_2d(ctx, qkv, Nkv * D, N, qkv.contents.nb[1], Nh * D * 4))
    q = L.ggml_reshape_3d(ctx, q, D, Nh, N)
    k = L.ggml_reshape_3d(ctx, k, D, Nkv, N)
    q = L.ggml_rope_ext(ctx, q, pos, None, D, 2, 0, 1e6, 1.0, 0.0, 1.0, 0.0, 0.0)
    rp = q.contents.op_params
    assert rp[1] == D and rp[2] == 2
    assert math.isclose(np.array([rp[5]], np.int32).view(np.float32)[0], 1e6)
    k = L.ggml_cont(ctx, L.ggml_rope_ext(ctx, k, pos, None, D, 2, 0, 1e6, 1.0, 0.0, 1.0, 0.0, 0.0))
    kset = L.ggml_view_4d(ctx, kc, D, S, Nkv, N, kc.contents.nb[1], kc.contents.nb[2], kc.contents.nb[3], 0)
    sr = L.ggml_set_rows(ctx, kset, L.ggml_reshape_4d(ctx, k, D, 1, Nkv, N), rows)
    L.ggml_build_forward_expand(gf, sr)
    kb = L.ggml_view_4d(ctx, kc, D, pad, Nkv, N, kc.contents.nb[1], kc.contents.nb[2], kc.contents.nb[3], 0)
    q4 = L.ggml_reshape_4d(ctx, L.ggml_cont(ctx, q), D, 1, Nh, N)
    fa = L.ggml_flash_attn_ext(ctx, q4, kb, kb, mask, 1 / math.sqrt(D), 0.0, 0.0)
    L.ggml_flash_attn_ext_set_prec(fa, 10)
    assert list(fa.contents.ne) == [D, Nh, 1, N]
    assert fa.contents.op_params[3] == 10
    L.ggml_build_forward_expand(gf, fa)
    names = [L.ggml_op_name(L.ggml_graph_node(gf, i).contents.op).decode() for i in range(L.ggml_graph_n_nodes(gf))]
    assert names.index("SET_ROWS") < names.index("FLASH_ATTN_EXT")
    assert names.count("MUL_MAT") == 1 and names.count("ROPE") == 2
    assert L.ggml_graph_n_leafs(gf) == 6  # x, wqkv, pos, rows, mask, cache
