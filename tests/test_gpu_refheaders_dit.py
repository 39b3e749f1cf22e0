"""GPU: the reference's own DiT code on the MI355X backend.

tests/refheaders/dit_driver (built from src/dit.h with src/gguf-weights.h,
src/weight-ctx.h and src/backend.h, unchanged) loads a GGUF this test writes
(DiT::load, src/dit.h:104-140: Q4_K block projections, proj_in, proj_out and
timestep MLP as the Q4_K_M preset stores them; F32 norms, biases, Fourier
weights and the two k=1 conv weights, which the quantiser leaves unquantised
since their ne0 is the kernel width 1) and runs DiT::forward
(src/dit.h:315-388) at the model's shape, T = 689 latent frames and CFG
batch B = 2: the graph of dit_build_graph (:249-287, 36 blocks between the
concat head and the proj_out / postprocess_conv tail) through
ggml_backend_sched_graph_compute, five times on the same inputs (eager, HIP
graph captured, then replayed, with the backend's f16 weight copies made on
the third sight).

The restatement is float32 torch on the CPU with the weights dequantised by
the oracle; the attention rounds K and V to f16 as the graph's casts do
(src/dit.h:219-220).  Stated tolerances, per probe: cosine >= 0.9999 and
relative RMS error <= 5e-3, for
- the head: hidden_after_preprocess, hidden_after_proj_in, the timestep row
  (computed on the host by the reference itself, max-rel 1e-4);
- every block, teacher-forced: the restatement of block l starts from the
  GPU's own input of that block, so no earlier difference is carried in;
- the named probes (layer0_sa_output, hidden_after_layer0/6/12/18/35) and
  the velocity against the restatement chained from the inputs alone;
- the tail (proj_out, postprocess_conv + residual) from the GPU's own last
  block output.
All five runs give the same velocity bit for bit; the driver's host-clock
time per DiT::forward is printed."""
import concurrent.futures
import ctypes
import json
import os
import pathlib
import subprocess

import numpy as np
import pytest
import torch

import gguf_writer
from conftest import cosine

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parent.parent
DRIVER = ROOT / "tests" / "refheaders" / "_build" / "dit_driver"
DIM, IN_CH, COND, CONCAT, NL = 2048, 128, 2048, 2304, 36
NH, HD, FF, ROT, FOURIER = 32, 64, 8192, 32, 256
LN_EPS, ROPE_BASE = 1e-5, 10000.0
Q4_K, F32 = 12, 0
PROBES = (0, 6, 12, 18, NL - 1)


def _q4_k(rng, n, k, gain=1.0):
    """GGUF Q4_K rows [n, k]: random quants, 6-bit scales and mins, d and dmin
    chosen so that w = d*sc*q - dmin*m has mean ~0 and standard deviation
    ~gain / sqrt(k) (d*sc*q has standard deviation ~258 d for uniform sc, m,
    q; dmin = 7.5 d centres it)."""
    nb = n * k // 256
    blk = rng.integers(0, 1 << 63, size=nb * 18, dtype=np.uint64).view(np.uint8).reshape(nb, 144)
    s = gain / np.sqrt(k) / 258.0
    d = (s * rng.uniform(0.5, 1.5, nb)).astype(np.float16)
    dmin = (7.5 * s * rng.uniform(0.5, 1.5, nb)).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def _model(seed):
    """{gguf name: (ggml type, ne, array)} of a DiT with the reference's
    tensor names and shapes (src/dit.h:16-21, :118-140)."""
    rng = np.random.default_rng(seed)

    def f32(*shape, scale=1.0, mean=0.0):
        return (mean + scale * rng.standard_normal(shape)).astype(np.float32)

    w = {
        "time_proj.weight": (F32, [128], f32(128)),
        "time_embed.linear_1.weight": (Q4_K, [FOURIER, DIM], _q4_k(rng, DIM, FOURIER)),
        "time_embed.linear_1.bias": (F32, [DIM], f32(DIM, scale=0.02)),
        "time_embed.linear_2.weight": (Q4_K, [DIM, DIM], _q4_k(rng, DIM, DIM)),
        "time_embed.linear_2.bias": (F32, [DIM], f32(DIM, scale=0.02)),
        # k = 1 convs [out, in, 1] in torch order: ne = [1, in, out]
        "preprocess_conv.weight": (F32, [1, CONCAT, CONCAT], f32(CONCAT, CONCAT, scale=1 / np.sqrt(CONCAT))),
        "proj_in.weight": (Q4_K, [CONCAT, DIM], _q4_k(rng, DIM, CONCAT)),
        "proj_out.weight": (Q4_K, [DIM, IN_CH], _q4_k(rng, IN_CH, DIM)),
        "postprocess_conv.weight": (F32, [1, IN_CH, IN_CH], f32(IN_CH, IN_CH, scale=1 / np.sqrt(IN_CH))),
    }
    for i in range(NL):
        p = f"transformer_blocks.{i}."
        w.update({
            p + "norm1.weight": (F32, [DIM], f32(DIM, scale=0.05, mean=1.0)),
            p + "norm1.bias": (F32, [DIM], f32(DIM, scale=0.02)),
            p + "attn.to_q.weight": (Q4_K, [DIM, DIM], _q4_k(rng, DIM, DIM)),
            p + "attn.to_k.weight": (Q4_K, [DIM, DIM], _q4_k(rng, DIM, DIM)),
            p + "attn.to_v.weight": (Q4_K, [DIM, DIM], _q4_k(rng, DIM, DIM)),
            p + "attn.to_out.0.weight": (Q4_K, [DIM, DIM], _q4_k(rng, DIM, DIM)),
            p + "norm2.weight": (F32, [DIM], f32(DIM, scale=0.05, mean=1.0)),
            p + "norm2.bias": (F32, [DIM], f32(DIM, scale=0.02)),
            p + "ff_in.weight": (Q4_K, [DIM, 2 * FF], _q4_k(rng, 2 * FF, DIM)),
            p + "ff_in.bias": (F32, [2 * FF], f32(2 * FF, scale=0.02)),
            p + "ff_out.weight": (Q4_K, [FF, DIM], _q4_k(rng, DIM, FF)),
            p + "ff_out.bias": (F32, [DIM], f32(DIM, scale=0.02)),
        })
    return w


class _Ref:
    """Float32 restatement of src/dit.h on the CPU (torch), weights
    dequantised by the oracle (its Q4_K rows, threaded over row ranges)."""

    def __init__(self, orc, w):
        self.orc, self.w = orc, w
        self.nt = orc.default_threads()
        torch.set_num_threads(self.nt)
        self.pool = concurrent.futures.ThreadPoolExecutor(self.nt)

    def mat(self, name):
        """[out, in] float32 torch matrix of a weight."""
        t, ne, a = self.w[name]
        k, n = (ne[0], ne[1]) if len(ne) == 2 else (ne[1], ne[2])
        if t == F32:
            return torch.from_numpy(np.ascontiguousarray(a).reshape(n, k))
        out = np.empty((n, k), np.float32)
        rs = k // 256 * 144
        step = max(1, (n + self.nt - 1) // self.nt)
        L = self.orc.lib()

        def part(r0):
            r1 = min(n, r0 + step)
            L.orc_dequantize_row(t, ctypes.c_void_p(a.ctypes.data + r0 * rs),
                                 ctypes.c_void_p(out.ctypes.data + r0 * k * 4), (r1 - r0) * k)

        list(self.pool.map(part, range(0, n, step)))
        return torch.from_numpy(out)

    def vec(self, name):
        return torch.from_numpy(self.w[name][2])

    def temb(self, t):
        """dit_time_embed (src/dit.h:289-313) in float64."""
        f = self.w["time_proj.weight"][2].astype(np.float64)
        ang = 2.0 * np.pi * t * f
        emb = np.concatenate([np.cos(ang), np.sin(ang)])
        h = self.mat("time_embed.linear_1.weight").double().numpy() @ emb + self.vec("time_embed.linear_1.bias").double().numpy()
        h = h / (1.0 + np.exp(-h))
        return self.mat("time_embed.linear_2.weight").double().numpy() @ h + self.vec("time_embed.linear_2.bias").double().numpy()

    def head(self, xt, cond, temb):
        """dit_build_graph up to the blocks (src/dit.h:252-268): returns
        (hidden_after_preprocess, hidden_after_proj_in, blocks' input)."""
        B, T, _ = xt.shape
        x = torch.cat([xt, torch.zeros(B, T, IN_CH), cond], dim=-1)
        x = x @ self.mat("preprocess_conv.weight").T + x
        p = x @ self.mat("proj_in.weight").T
        tok = torch.from_numpy(np.broadcast_to(temb.astype(np.float32), (B, 1, DIM)).copy())
        return x, p, torch.cat([tok, p], dim=1)

    def block(self, l, x, W):
        """dit_block (src/dit.h:183-247) on x [B, S, DIM]; returns (sa_out, out)."""
        B, S, _ = x.shape
        pre = f"transformer_blocks.{l}."
        h = _ln(x, self.vec(pre + "norm1.weight"), self.vec(pre + "norm1.bias"))
        q = (h @ W["q"].T).reshape(B, S, NH, HD)
        k = (h @ W["k"].T).reshape(B, S, NH, HD)
        v = (h @ W["v"].T).reshape(B, S, NH, HD)
        pos = torch.arange(S)
        q = _rope(q, pos)
        k = _rope(k, pos).half().float()
        v = v.half().float()
        qh, kh, vh = (a.permute(0, 2, 1, 3).contiguous() for a in (q, k, v))
        p = torch.softmax((qh @ kh.transpose(-1, -2).contiguous()) / np.sqrt(HD), dim=-1)
        a = (p @ vh).permute(0, 2, 1, 3).reshape(B, S, NH * HD)
        sa = a @ W["o"].T
        x = x + sa
        h = _ln(x, self.vec(pre + "norm2.weight"), self.vec(pre + "norm2.bias"))
        f = h @ W["ff_in"].T + self.vec(pre + "ff_in.bias")
        value, gate = f[..., :FF], f[..., FF:]
        return sa, x + (torch.nn.functional.silu(gate) * value) @ W["ff_out"].T + self.vec(pre + "ff_out.bias")

    def block_weights(self, l):
        pre = f"transformer_blocks.{l}."
        names = dict(q="attn.to_q.weight", k="attn.to_k.weight", v="attn.to_v.weight", o="attn.to_out.0.weight",
                     ff_in="ff_in.weight", ff_out="ff_out.weight")
        return {k: self.mat(pre + n) for k, n in names.items()}

    def tail(self, x):
        """src/dit.h:280-286 on the last block's output x [B, T + 1, DIM]:
        (proj_out output, velocity)."""
        y = x[:, 1:].contiguous() @ self.mat("proj_out.weight").T
        return y, y @ self.mat("postprocess_conv.weight").T + y


def _ln(x, w, b):
    m = x.mean(-1, keepdim=True)
    v = ((x - m) ** 2).mean(-1, keepdim=True)
    return (x - m) / torch.sqrt(v + LN_EPS) * w + b


def _rope(x, pos):
    """x [B, S, H, D]: NeoX pairs (i, i + ROT/2) of the first ROT dims rotate
    by pos * base^(-2i/ROT) (the remaining dims pass through)."""
    half = ROT // 2
    inv = ROPE_BASE ** (-2.0 * torch.arange(half, dtype=torch.float64) / ROT)
    ang = (pos.to(torch.float64)[:, None] * inv[None, :]).to(torch.float32)
    c, s = torch.cos(ang)[None, :, None, :], torch.sin(ang)[None, :, None, :]
    y = x.clone()
    x0, x1 = x[..., :half], x[..., half:ROT]
    y[..., :half] = x0 * c - x1 * s
    y[..., half:ROT] = x0 * s + x1 * c
    return y


def _relrms(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.sqrt(np.mean((a - b) ** 2) / np.mean(b * b)))


def _close(what, a, ref):
    c, r = cosine(a, ref), _relrms(a, ref)
    print(f"{what}: cosine {c:.7f}, rel-RMS {r:.2e}", flush=True)
    assert c >= 0.9999 and r <= 5e-3, (what, c, r)


@pytest.mark.timeout(600)
def test_reference_dit_runs_on_the_backend(orc, tmp_path):
    assert DRIVER.exists(), f"{DRIVER} is not built"
    T, B, t, runs = 689, 2, 0.37, 5
    S = T + 1
    w = _model(61)
    gguf_writer.write(tmp_path / "dit.gguf", [], [(n, ty, ne, a) for n, (ty, ne, a) in w.items()])
    rng = np.random.default_rng(62)
    xt = rng.standard_normal((B, T, IN_CH)).astype(np.float32)
    cond = rng.standard_normal((B, T, COND)).astype(np.float32)
    xt.tofile(tmp_path / "xt.bin")
    cond.tofile(tmp_path / "cond.bin")

    print(f"running the reference DiT driver: T={T} B={B} t={t}, {runs} runs", flush=True)
    env = dict(os.environ, GGML_BACKEND="MI355X0")
    r = subprocess.run([str(DRIVER), str(tmp_path / "dit.gguf"), str(tmp_path), str(T), str(B), str(t), str(runs)],
                       capture_output=True, text=True, timeout=280, env=env)
    print(r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stderr[-3000:]
    info = json.loads(r.stdout.strip().splitlines()[-1])
    print(info, flush=True)
    (tmp_path / "dit.gguf").unlink()
    assert info["backend"] == "MI355X0" and info["runs_identical"] and info["replays"] >= 1
    print(f"DiT::forward at T={T}, B={B}: {min(info['ms'][2:]):.2f} ms per step (best of the replays; "
          f"first, eager: {info['ms'][0]:.1f} ms)", flush=True)

    vel = np.fromfile(tmp_path / "velocity.bin", np.float32).reshape(B, T, IN_CH)
    assert np.array_equal(vel, np.fromfile(tmp_path / "velocity_last.bin", np.float32).reshape(B, T, IN_CH))
    assert np.isfinite(vel).all()
    hb = np.fromfile(tmp_path / "head.bin", np.float32)
    n_pre, n_in, n_x = B * T * CONCAT, B * T * DIM, B * S * DIM
    g_pre = hb[:n_pre].reshape(B, T, CONCAT)
    g_pin = hb[n_pre:n_pre + n_in].reshape(B, T, DIM)
    g_x0 = hb[n_pre + n_in:n_pre + n_in + n_x].reshape(B, S, DIM)
    g_sa0 = hb[n_pre + n_in + n_x:].reshape(B, S, DIM)
    blocks = np.memmap(tmp_path / "blocks.bin", np.float32, "r", shape=(NL, B, S, DIM))
    g_y = np.fromfile(tmp_path / "tail.bin", np.float32).reshape(B, T, IN_CH)

    ref = _Ref(orc, w)
    temb = ref.temb(t)
    err = np.abs(g_x0[:, 0] - temb[None].astype(np.float32)).max() / np.abs(temb).max()
    print(f"timestep token (host, dit_time_embed): max-rel {err:.2e}", flush=True)
    assert err <= 1e-4
    r_pre, r_pin, r_x = ref.head(torch.from_numpy(xt), torch.from_numpy(cond), temb)
    _close("hidden_after_preprocess", g_pre, r_pre.numpy())
    _close("hidden_after_proj_in", g_pin, r_pin.numpy())

    with torch.no_grad():
        for l in range(NL):
            W = ref.block_weights(l)
            g_in = torch.from_numpy(np.array(g_x0 if l == 0 else blocks[l - 1]))
            sa, tf = ref.block(l, g_in, W)  # teacher-forced
            _close(f"block {l} (teacher-forced)", blocks[l], tf.numpy())
            if l == 0:
                _close("layer0_sa_output (teacher-forced)", g_sa0, sa.numpy())
            sa, r_x = ref.block(l, r_x, W)  # chained from the inputs
            if l == 0:
                _close("layer0_sa_output (chained)", g_sa0, sa.numpy())
            if l in PROBES:
                _close(f"hidden_after_layer{l} (chained)", blocks[l], r_x.numpy())
        y, v = ref.tail(torch.from_numpy(np.array(blocks[NL - 1])))
        _close("proj_out (from the GPU's last block)", g_y, y.numpy())
        _close("velocity (from the GPU's proj_out)", vel, (torch.from_numpy(g_y) @ ref.mat("postprocess_conv.weight").T
                                                          + torch.from_numpy(g_y)).numpy())
        _close("velocity (from the GPU's last block)", vel, v.numpy())
        _, v = ref.tail(r_x)
        _close("velocity (chained)", vel, v.numpy())
