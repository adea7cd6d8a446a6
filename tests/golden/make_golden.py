"""Writes tests/golden/golden.npz: seeded small inputs of the quantized attention path and the oracle's outputs
for them. Run from the repository root: `python tests/golden/make_golden.py`.

Cases (bf16 inputs stored as their 16-bit patterns, int16):
  requant : K, V [1, 100, 2, 128] (K with a per-channel offset)   -> k8, k_scale, km, v8, v8lo, v_scale
  quant_q : Q [1, 70, 2, 128]                                     -> q8, q_scale
  logits  : q8 x k8 of the two cases above                        -> int32 [2, 256, 100]
  attn1   : Q [1, 70, 2, 128] over the requant chunk              -> fp32 out [70, 2, 128]
  ring    : Q [1, 70, 2, 128] over chunks of 90, 64 and 100 keys  -> fp32 out [70, 2, 128]
The attention outputs follow the kernel's schedule for 32 persistent workgroups per XCD (256 CUs)."""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import emu  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
GX = 32


def bits(x):
    return x.contiguous().view(torch.int16).numpy()


def make():
    g = torch.Generator().manual_seed(2024)
    h = 2

    def randn(*shape, scale=1.0):
        return torch.randn(*shape, generator=g) * scale

    k = (randn(1, 100, h, 128) + randn(1, 1, h, 128, scale=3.0)).to(torch.bfloat16)
    v = randn(1, 100, h, 128, scale=1.7).to(torch.bfloat16)
    q = randn(1, 70, h, 128, scale=2.0).to(torch.bfloat16)
    mem = [((randn(1, n, h, 128) + randn(1, 1, h, 128, scale=3.0)).to(torch.bfloat16),
            randn(1, n, h, 128, scale=1.5).to(torch.bfloat16)) for n in (90, 64)]

    r = emu.requant(k, v)
    q8, qs = emu.quant_q(q)
    out = {
        "k": bits(k), "v": bits(v), "q": bits(q),
        "mem0_k": bits(mem[0][0]), "mem0_v": bits(mem[0][1]), "mem1_k": bits(mem[1][0]), "mem1_v": bits(mem[1][1]),
        "k8": r["k8"].numpy(), "k_scale": r["k_scale"].numpy(), "km": r["km"].numpy(),
        "v8": r["v8"].numpy(), "v8lo": r["v8lo"].numpy(), "v_scale": r["v_scale"].numpy(),
        "q8": q8.numpy(), "q_scale": qs.numpy(),
        "logits": emu.qk_logits(q8, r["k8"])[:, :, :100].numpy(),
        "attn1": emu.attention(q, [r], schedule_gx=GX).numpy(),
        "ring": emu.attention(q, [emu.requant(mk, mv) for mk, mv in mem] + [r], schedule_gx=GX).numpy(),
        "gx": np.array(GX),
    }
    return out


def load(path=OUT):
    """The fixture as {name: numpy array}, with the bf16 inputs back as torch bf16 tensors."""
    with np.load(path, allow_pickle=False) as z:
        d = {name: z[name] for name in z.files}
    for name in ("k", "v", "q", "mem0_k", "mem0_v", "mem1_k", "mem1_v"):
        d[name] = torch.from_numpy(d[name]).view(torch.bfloat16)
    return d


if __name__ == "__main__":
    np.savez_compressed(OUT, **make())
    print(OUT, os.path.getsize(OUT), "bytes")
