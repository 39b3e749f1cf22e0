"""Minimal GGUF v3 writer (test infrastructure): key-value pairs of the
scalar / string types and tensors as raw ggml bytes, in the layout the GGUF
reader of minimaxmusic.cpp_amd/ggml/src/gguf.cpp parses (magic, version, tensor
and key-value counts, key-value pairs, tensor infos with data offsets relative
to the aligned data section, padding, data)."""
import struct

GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, GGUF_BOOL, GGUF_STRING = 4, 5, 6, 7, 8


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, vtype, value):
    out = _str(key) + struct.pack("<I", vtype)
    if vtype == GGUF_STRING:
        return out + _str(value)
    fmt = {GGUF_UINT32: "<I", GGUF_INT32: "<i", GGUF_FLOAT32: "<f", GGUF_BOOL: "<?"}[vtype]
    return out + struct.pack(fmt, value)


def write(path, kvs, tensors, alignment=32):
    """kvs: [(key, gguf type, value)]; tensors: [(name, ggml type, ne list
    (ne[0] innermost), raw bytes)]."""
    head = b"GGUF" + struct.pack("<IqQ", 3, len(tensors), len(kvs))
    head += b"".join(_kv(k, t, v) for k, t, v in kvs)
    infos, offset, blobs = [], 0, []
    for name, gtype, ne, data in tensors:
        data = memoryview(data)  # raw bytes of any buffer; contiguous ones are not copied
        data = data.cast("B") if data.c_contiguous else memoryview(data.tobytes())
        infos.append(_str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<q", int(n)) for n in ne))
        infos.append(struct.pack("<IQ", gtype, offset))
        pad = (-data.nbytes) % alignment
        blobs.append((data, pad))
        offset += data.nbytes + pad
    body = head + b"".join(infos)
    body += b"\0" * ((-len(body)) % alignment)
    with open(path, "wb") as f:
        f.write(body)
        for data, pad in blobs:
            f.write(data)
            f.write(b"\0" * pad)
