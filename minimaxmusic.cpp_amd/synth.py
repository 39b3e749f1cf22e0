"""Seeded synthetic GGUF weights and activations of the benchmark shapes.

No checkpoint is available offline, so weights are random blocks with the
distributions used for every measurement here:

* Q8_0: quants uniform in [-127, 127]; d = f16(|N(0, 0.02)| / 127).
* Q4_K: 4-bit quants and 6-bit (scale, min) pairs uniform (random bytes);
  d, dmin = f16(|N(0, 0.02)|).
* Q5_K: quant, fifth-bit and 6-bit (scale, min) bytes uniform;
  d = f16(|N(0, 0.02)| / 512), dmin = f16(|N(0, 0.02)| / 32), so that
  E[d sc q] = E[dmin m] (blocks centred on zero) and |w| ~ 0.01 like real
  weights and like the Q6_K blocks it is mixed with in the "_M" files.
* Q6_K: low/high quant bits uniform (random bytes); int8 scales uniform in
  [-64, 63]; d = f16(|N(0, 0.02)| / 1024), so |w| ~ 0.01 like real weights.

``*_np`` build host numpy bytes (parity tests); ``gguf_blocks_torch`` builds
the same distributions directly in device memory (large benchmarks).
"""
import numpy as np

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
# byte offset of the f16 scale fields inside each GGUF block
_D_FIELDS = {Q8_0: [0], Q4_K: [0, 2], Q5_K: [0, 2], Q6_K: [208]}
_DMIN_DIV = {Q4_K: (1.0, 1.0), Q5_K: (512.0, 32.0)}


def _scale_bits(rng, n, div):
    return (np.abs(rng.normal(0.0, 0.02, n)) / div).astype(np.float16).view(np.uint16)


def gguf_blocks_np(qtype, N, K, seed):
    be, bb = BLOCK[qtype]
    assert K % be == 0
    rng = np.random.default_rng(seed)
    nb = N * (K // be)
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if qtype == Q8_0:
        q = rng.integers(-127, 128, size=(nb, 32), dtype=np.int16).astype(np.int8)
        blk[:, 2:34] = q.view(np.uint8)
        d = _scale_bits(rng, nb, 127.0)
        blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    elif qtype in (Q4_K, Q5_K):
        dd, dm = _DMIN_DIV[qtype]
        blk[:, 0:2] = _scale_bits(rng, nb, dd).view(np.uint8).reshape(nb, 2)
        blk[:, 2:4] = _scale_bits(rng, nb, dm).view(np.uint8).reshape(nb, 2)
    elif qtype == Q6_K:
        sc = rng.integers(-64, 64, size=(nb, 16), dtype=np.int16).astype(np.int8)
        blk[:, 192:208] = sc.view(np.uint8)
        blk[:, 208:210] = _scale_bits(rng, nb, 1024.0).view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def gguf_blocks_torch(qtype, N, K, seed, device="cuda"):
    """Same distributions, generated on the device (uint8 GGUF bytes)."""
    import torch

    be, bb = BLOCK[qtype]
    assert K % be == 0
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    nb = N * (K // be)
    blk = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device=device, generator=g)

    def scale(div):
        return (torch.randn(nb, device=device, generator=g) * 0.02).abs_().div_(div).to(torch.float16).view(torch.uint8).view(nb, 2)

    if qtype == Q8_0:
        q = torch.randint(-127, 128, (nb, 32), dtype=torch.int8, device=device, generator=g)
        blk[:, 2:34] = q.view(torch.uint8)
        blk[:, 0:2] = scale(127.0)
    elif qtype in (Q4_K, Q5_K):
        dd, dm = _DMIN_DIV[qtype]
        blk[:, 0:2] = scale(dd)
        blk[:, 2:4] = scale(dm)
    elif qtype == Q6_K:
        sc = torch.randint(-64, 64, (nb, 16), dtype=torch.int8, device=device, generator=g)
        blk[:, 192:208] = sc.view(torch.uint8)
        blk[:, 208:210] = scale(1024.0)
    return blk.view(-1)


def normal_np(shape, seed, dtype=np.float32):
    return np.random.default_rng(seed).standard_normal(shape).astype(dtype)
