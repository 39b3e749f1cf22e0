"""GPU: mmhip_flash_attn_ext_noalloc (the attention entry point that
allocates nothing: its workspace is a file-scope device array) against
mmhip_flash_attn_ext with a caller-allocated workspace, bit for bit, on two
calls in a row with the second smaller, for the split-KV decode kernels and
for the masked MFMA kernel (whose mask prepass uses the scratch)."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, D, nq, nkv, seed, mask_kind):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, Hq, nq, D), generator=g).cuda()
    k = torch.randn((B, Hkv, nkv, D), generator=g).half().cuda()
    v = torch.randn((B, Hkv, nkv, D), generator=g).half().cuda()
    mask = None
    if mask_kind == "pad":  # the decode graph's padded window: 0 up to the length, -inf after
        m = torch.zeros((1, 1, nq, nkv), dtype=torch.float16)
        m[..., nkv - 256:] = float("-inf")
        mask = m.cuda()
    elif mask_kind == "causal":
        m = torch.triu(torch.full((nq, nkv), float("-inf")), 1).half().reshape(1, 1, nq, nkv)
        mask = m.cuda()
    return q, k, v, mask


def _noalloc(mm, q, k, v, mask, scale):
    B, Hq, nq, D = q.shape
    out = torch.empty((B, nq, Hq, D), dtype=torch.float32, device=q.device)
    qv, kv, vv = mm.view_of(q), mm.view_of(k), mm.view_of(v)
    mv = mm.view_of(mask) if mask is not None else None
    rc = mm.load().mmhip_flash_attn_ext_noalloc(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv),
                                                 ctypes.byref(mv) if mv is not None else None, scale,
                                                 ctypes.c_void_p(out.data_ptr()),
                                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, mm.load().mmhip_last_error()
    return out


@pytest.mark.parametrize("shapes", [
    # split-KV decode (MFMA decode kernel, partials in the scratch), then smaller
    [(2, 32, 8, 128, 1, 2304, "pad"), (1, 16, 4, 64, 1, 700, None)],
    # masked MFMA attention (row-end prepass in the scratch), then smaller
    [(1, 8, 2, 128, 512, 512, "causal"), (1, 4, 2, 64, 200, 200, "causal")],
])
def test_noalloc_matches_workspace_entry(mm, shapes):
    L = mm.load()
    assert L.mmhip_flash_attn_noalloc_max_workspace() == 8 << 20
    for i, (B, Hq, Hkv, D, nq, nkv, mk) in enumerate(shapes):
        print(f"noalloc case {i}: B={B} Hq={Hq} Hkv={Hkv} D={D} nq={nq} nkv={nkv} mask={mk}", flush=True)
        q, k, v, mask = _inputs(B, Hq, Hkv, D, nq, nkv, 100 + i, mk)
        scale = 1.0 / np.sqrt(D)
        qv, kv, vv = mm.view_of(q), mm.view_of(k), mm.view_of(v)
        need = L.mmhip_flash_attn_workspace(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv))
        assert 0 < need <= 8 << 20
        ref = mm.flash_attn_ext(q, k, v, mask, scale)
        got = _noalloc(mm, q, k, v, mask, scale)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        assert torch.isfinite(got).all()
