"""Host-side checks of the restated GGUF reader (gguf.h) and of the host
decoders behind ggml_get_type_traits(t)->to_float, which the reference's
weight loader uses (src/gguf-weights.h:76-203, :230-283).  No GPU needed.

- The reader returns the key-value pairs, tensor names, types, shapes and
  data offsets a file written by tests/gguf_writer.py holds (data compared
  byte for byte at data_offset + offset), creates the descriptor context with
  and without data, honours general.alignment, and refuses a truncated file.
- to_float is bit-exact against the oracle's dequantisation (itself pinned to
  the golden known-answer blocks) for Q8_0 / Q4_K / Q6_K, and equal to
  numpy's conversion for F16 and BF16.
"""
import ctypes

import numpy as np
import pytest

import ggml_ctypes as G
import gguf_writer

F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30


class GgufInit(ctypes.Structure):
    _fields_ = [("no_alloc", ctypes.c_bool), ("ctx", ctypes.POINTER(ctypes.c_void_p))]


class TypeTraits(ctypes.Structure):
    _fields_ = [("type_name", ctypes.c_char_p), ("blck_size", ctypes.c_int64), ("blck_size_interleave", ctypes.c_int64),
                ("type_size", ctypes.c_size_t), ("is_quantized", ctypes.c_bool), ("to_float", ctypes.c_void_p),
                ("from_float_ref", ctypes.c_void_p)]


TO_FLOAT = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64)


@pytest.fixture(scope="module")
def L():
    import __graft_entry__

    if not G.LIB.exists():
        __graft_entry__.build()
    L = G.load()
    vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
    for n, r, a in [("gguf_init_from_file", vp, [ctypes.c_char_p, GgufInit]), ("gguf_free", None, [vp]),
                    ("gguf_get_n_tensors", i64, [vp]), ("gguf_get_n_kv", i64, [vp]),
                    ("gguf_find_tensor", i64, [vp, ctypes.c_char_p]), ("gguf_find_key", i64, [vp, ctypes.c_char_p]),
                    ("gguf_get_tensor_offset", sz, [vp, i64]), ("gguf_get_tensor_name", ctypes.c_char_p, [vp, i64]),
                    ("gguf_get_tensor_type", ctypes.c_int, [vp, i64]), ("gguf_get_tensor_size", sz, [vp, i64]),
                    ("gguf_get_data_offset", sz, [vp]), ("gguf_get_alignment", sz, [vp]),
                    ("gguf_get_val_str", ctypes.c_char_p, [vp, i64]), ("gguf_get_val_u32", ctypes.c_uint32, [vp, i64]),
                    ("gguf_get_val_f32", ctypes.c_float, [vp, i64]), ("gguf_get_kv_type", ctypes.c_int, [vp, i64]),
                    ("ggml_get_tensor", G.T, [vp, ctypes.c_char_p]),
                    ("ggml_get_type_traits", ctypes.POINTER(TypeTraits), [ctypes.c_int])]:
        fn = getattr(L, n)
        fn.restype, fn.argtypes = r, a
    return L


def _tensors(pkg):
    rng = np.random.default_rng(3)
    return [("a.q8", Q8_0, [256, 5], pkg.synth.gguf_blocks_np(Q8_0, 5, 256, 1)),
            ("b.norm", F32, [300], rng.standard_normal(300).astype(np.float32)),
            ("c.q6", Q6_K, [512, 3], pkg.synth.gguf_blocks_np(Q6_K, 3, 512, 2)),
            ("d.cube", F16, [4, 3, 2], rng.standard_normal(24).astype(np.float16).view(np.uint8))]


@pytest.mark.parametrize("alignment", [32, 256])
def test_gguf_reader_roundtrip(L, pkg, tmp_path, alignment):
    path = tmp_path / "m.gguf"
    tensors = _tensors(pkg)
    kvs = [("mm3.config_json", gguf_writer.GGUF_STRING, '{"hidden_size": 256}'),
           ("general.alignment", gguf_writer.GGUF_UINT32, alignment),
           ("x.scale", gguf_writer.GGUF_FLOAT32, 0.5)]
    gguf_writer.write(path, kvs, tensors, alignment=alignment)
    raw = path.read_bytes()
    for no_alloc in (True, False):
        meta = ctypes.c_void_p()
        g = L.gguf_init_from_file(str(path).encode(), GgufInit(no_alloc, ctypes.pointer(meta)))
        assert g and meta
        try:
            assert L.gguf_get_n_tensors(g) == 4 and L.gguf_get_n_kv(g) == 3
            assert L.gguf_get_alignment(g) == alignment
            assert L.gguf_get_val_str(g, L.gguf_find_key(g, b"mm3.config_json")) == b'{"hidden_size": 256}'
            assert L.gguf_get_val_f32(g, L.gguf_find_key(g, b"x.scale")) == 0.5
            assert L.gguf_find_key(g, b"nope") == -1 and L.gguf_find_tensor(g, b"nope") == -1
            base = L.gguf_get_data_offset(g)
            assert base % alignment == 0
            for name, gtype, ne, data in tensors:
                i = L.gguf_find_tensor(g, name.encode())
                assert L.gguf_get_tensor_name(g, i) == name.encode() and L.gguf_get_tensor_type(g, i) == gtype
                off = L.gguf_get_tensor_offset(g, i)
                data = bytes(data)
                assert off % alignment == 0 and L.gguf_get_tensor_size(g, i) == len(data)
                assert raw[base + off:base + off + len(data)] == data
                t = L.ggml_get_tensor(meta, name.encode())
                assert t and t.contents.type == gtype
                assert list(t.contents.ne) == list(ne) + [1] * (4 - len(ne))
                if no_alloc:
                    assert not t.contents.data
                else:
                    assert ctypes.string_at(t.contents.data, len(data)) == data
        finally:
            L.gguf_free(g)
            L.ggml_free(meta)


def test_gguf_reader_refuses_bad_files(L, pkg, tmp_path):
    path = tmp_path / "m.gguf"
    gguf_writer.write(path, [("k", gguf_writer.GGUF_UINT32, 1)], _tensors(pkg))
    raw = path.read_bytes()
    bad = tmp_path / "bad.gguf"
    for cut in (3, 20, 60):  # inside the magic, the counts, the key-value pairs
        bad.write_bytes(raw[:cut])
        assert not L.gguf_init_from_file(str(bad).encode(), GgufInit(True, None))
    bad.write_bytes(b"GGML" + raw[4:])
    assert not L.gguf_init_from_file(str(bad).encode(), GgufInit(True, None))
    # the header parses but the data section is cut: no data context
    bad.write_bytes(raw[:len(raw) - 100])
    meta = ctypes.c_void_p()
    assert not L.gguf_init_from_file(str(bad).encode(), GgufInit(False, ctypes.pointer(meta)))


def test_gguf_reader_refuses_overflowing_sizes(L, tmp_path):
    """Tensor shapes whose element count passes INT64_MAX, or whose byte size
    passes SIZE_MAX, are refused whether data is requested or not (a wrapped
    size would size the data context too small for the read)."""
    bad = tmp_path / "huge.gguf"
    for ne in ([32, 1 << 40, 1 << 40], [1 << 31, 1 << 31, 4], [256, 1 << 30, 1 << 30, 1 << 10], [256, 1 << 54]):
        gguf_writer.write(bad, [], [("huge", F32, ne, np.zeros(8, np.float32))])
        for no_alloc in (True, False):
            meta = ctypes.c_void_p()
            assert not L.gguf_init_from_file(str(bad).encode(), GgufInit(no_alloc, ctypes.pointer(meta))), (ne, no_alloc)
    # large but representable: the header parses, the data cannot be in the file
    gguf_writer.write(bad, [], [("big", F32, [256, 1 << 50], np.zeros(8, np.float32))])
    meta = ctypes.c_void_p()
    g = L.gguf_init_from_file(str(bad).encode(), GgufInit(True, ctypes.pointer(meta)))
    assert g
    L.gguf_free(g)
    L.ggml_free(meta)
    assert not L.gguf_init_from_file(str(bad).encode(), GgufInit(False, ctypes.pointer(meta)))


@pytest.mark.parametrize("gtype,K", [(Q8_0, 512), (Q4_K, 512), (Q6_K, 768)])
def test_to_float_matches_oracle(L, pkg, orc, gtype, K):
    rows = 7
    blocks = pkg.synth.gguf_blocks_np(gtype, rows, K, 11 + gtype)
    tr = L.ggml_get_type_traits(gtype).contents
    assert tr.is_quantized and tr.to_float
    fn = TO_FLOAT(tr.to_float)
    out = np.empty(rows * K, np.float32)
    fn(blocks.ctypes.data, out.ctypes.data, rows * K)
    ref = orc.dequantize(gtype, blocks, K, rows).reshape(-1)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_to_float_f16_bf16(L):
    x = np.random.default_rng(5).standard_normal(1000).astype(np.float32)
    out = np.empty(1000, np.float32)
    h = x.astype(np.float16)
    TO_FLOAT(L.ggml_get_type_traits(F16).contents.to_float)(h.ctypes.data, out.ctypes.data, 1000)
    assert np.array_equal(out, h.astype(np.float32))
    b = (x.view(np.uint32) >> 16).astype(np.uint16)
    TO_FLOAT(L.ggml_get_type_traits(BF16).contents.to_float)(b.ctypes.data, out.ctypes.data, 1000)
    assert np.array_equal(out.view(np.uint32), b.astype(np.uint32) << 16)
    assert not L.ggml_get_type_traits(F32).contents.to_float


def test_reference_loader_on_host_standin(L, pkg, tmp_path):
    """The reference's qw3lm_load (src/qwen3-lm.h:290-343, through gf_load,
    the fused QKV / gate_up loads and wctx_alloc) run by tests/refheaders/
    lm_driver with GGML_BACKEND=CPU: the weights land in the host stand-in's
    buffers byte for byte as the GGUF holds them; the first forward then stops
    with the reference's FATAL exit, since the stand-in computes nothing."""
    import os
    import subprocess

    import test_gpu_refheaders as R

    if not R.DRIVER.exists():
        pytest.skip("tests/refheaders/_build/lm_driver is built by __graft_entry__.build() where the reference "
                    "tree is present")
    gg, _, refw = R._model(pkg, 7)
    gguf_writer.write(tmp_path / "lm.gguf", [("mm3.config_json", gguf_writer.GGUF_STRING, R._config_json())], gg)
    np.zeros(4, np.int32).tofile(tmp_path / "tokens0.bin")
    np.zeros(4, np.int32).tofile(tmp_path / "tokens1.bin")
    np.zeros((1, 2, R.CFG["hidden"]), np.float32).tofile(tmp_path / "embeds.bin")
    env = dict(os.environ, GGML_BACKEND="CPU", HIP_VISIBLE_DEVICES="-1")
    r = subprocess.run([str(R.DRIVER), str(tmp_path / "lm.gguf"), str(tmp_path), "1", str(R.CFG["max_seq"])],
                       capture_output=True, text=True, timeout=120, env=env)
    assert "LM backend: CPU" in r.stderr and "Q+K+V fused" in r.stderr and "gate+up fused" in r.stderr
    assert r.returncode == 1 and "failed to allocate graph (prefill" in r.stderr, r.stderr[-1500:]
    R._check_weights(tmp_path / "weights.bin", refw)
