"""CPU restatement of the self-attention prologue: RMSNorm of the q / k projections and the 3-axis rotary
embedding (the oracle for the fused norm + rope + quantise kernels; test infrastructure only).

The reference, per DiT block (lingbot/models/lingbot_world/transformer.py:199-212):
  q = norm_q(Wq x), k = norm_k(Wk x)    WanRMSNorm over all C = heads * 128 channels of a token
                                        (reference/wan/modules/model.py:70-86): bf16(x * rsqrt(mean(x^2) + eps))
                                        in fp32, then times the bf16 weight (a bf16 product)
  q, k = causal_rope_apply(q / k)       pairs (x[2j], x[2j+1]) rotated in fp64 by the angle of token t, pair j
                                        (transformer.py:134-146), cast back to bf16 (fp64 -> fp32 -> bf16, the
                                        way torch casts a double tensor to bfloat16)
The rotation table is the concatenation of three rope_params tables (reference/wan/modules/model.py:29-36;
transformer.py:553-556): 22 frame pairs, 21 height pairs, 21 width pairs for d = 128; token t of a chunk with
grid (F, H, W) starting at latent frame f0 takes frame row f0 + t // (H W), height row (t // W) % H and width
row t % W (causal_rope_freqs, transformer.py:53-77).

The reference sums mean(x^2) in fp32 in its library's order; here the order is fixed so the kernels can be
checked bit for bit. Token row x (C = heads * 128 channels), channel c = 128 h + 8 g + e (g in 0..15, e in 0..7):
  a[h, g] = (((0 + x[c0]^2) + x[c0+1]^2) + ... + x[c0+7]^2)           fp64, c0 = 128 h + 8 g
  P[h]    = pairwise over g: ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)), the same for 8..15, then the two halves added
  total   = ((0 + P[0]) + P[1]) + ... + P[heads - 1]                   fp64
  ms      = fp32(total / C);  r = fp32(1 / sqrt(fp64(ms + eps)))      (ms + eps an fp32 sum)
  y       = bf16(x * r) (fp32 product);  n = bf16(y * w)
Squares of bf16 values are exact in fp64 and the sum of 1536 of them nearly always is too, so the order rarely
matters; the fp64 reciprocal square root rounds to the same fp32 as the exact one except within 2^-29 of a
rounding boundary.
"""
import numpy as np
import torch

HEAD_DIM = 128


def rope_params(max_seq_len, dim, theta=10000):
    """Complex rotation table [max_seq_len, dim / 2]: angle t / theta^(2i / dim) (reference/wan/modules/model.py:29-36)."""
    assert dim % 2 == 0
    inv = 1.0 / torch.pow(torch.tensor(float(theta), dtype=torch.float64),
                          torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.outer(torch.arange(max_seq_len, dtype=torch.float64), inv)
    return torch.polar(torch.ones_like(ang), ang)


def rope_table(d=HEAD_DIM, rows=1024):
    """The model's (cos, sin) table, float64 [rows, d / 2, 2] (transformer.py:553-556)."""
    s = d // 6
    return torch.view_as_real(torch.cat([rope_params(rows, d - 4 * s), rope_params(rows, 2 * s),
                                         rope_params(rows, 2 * s)], dim=1)).contiguous()


def rope_sections(d=HEAD_DIM):
    """Pairs of the frame, height and width sections: [c - 2 (c // 3), c // 3, c // 3], c = d / 2."""
    c = d // 2
    return c - 2 * (c // 3), c // 3, c // 3


def rope_rows(n, grid_hw, start_frame, d=HEAD_DIM):
    """Table row of every (token, pair) of an n-token chunk: int64 [n, d / 2]."""
    gh, gw = grid_hw
    t = np.arange(n, dtype=np.int64)
    f, hh, ww = start_frame + t // (gh * gw), (t // gw) % gh, t % gw
    s0, s1, s2 = rope_sections(d)
    return np.concatenate([np.repeat(f[:, None], s0, 1), np.repeat(hh[:, None], s1, 1),
                           np.repeat(ww[:, None], s2, 1)], axis=1)


def rope_cos_sin(table, n, grid_hw, start_frame):
    """(cos, sin) float64 [n, d / 2] of an n-token chunk."""
    rows = torch.from_numpy(rope_rows(n, grid_hw, start_frame, 2 * table.shape[1]))
    j = torch.arange(table.shape[1])[None, :].expand(n, -1)
    return table[rows, j, 0], table[rows, j, 1]


def rms_norm(x, w, eps, heads):
    """x bf16 [L, C] (C = heads * 128), w bf16 [C] -> bf16 [L, C] in the order stated above."""
    L, C = x.shape
    assert C == heads * HEAD_DIM
    sq = x.double().pow(2).view(L, heads, 16, 8)
    a = torch.zeros(L, heads, 16, dtype=torch.float64)
    for e in range(8):
        a = a + sq[..., e]
    while a.shape[-1] > 1:
        a = a[..., 0::2] + a[..., 1::2]
    tot = torch.zeros(L, dtype=torch.float64)
    for h in range(heads):
        tot = tot + a[:, h, 0]
    ms = (tot / C).float()
    v = ms + torch.tensor(eps, dtype=torch.float32)
    r = (1.0 / torch.sqrt(v.double())).float()
    y = (x.float() * r[:, None]).to(torch.bfloat16)
    return (y.float() * w.float()[None, :]).to(torch.bfloat16)


def rope_apply(x, cos, sin):
    """x bf16 [L, H, 128], cos / sin float64 [L, 64] -> bf16 [L, H, 128] (fp64 rotation, products and sums
    rounded one at a time, then fp64 -> fp32 -> bf16)."""
    L, H, d = x.shape
    p = x.double().view(L, H, d // 2, 2)
    xr, xi = p[..., 0], p[..., 1]
    c, s = cos[:, None, :], sin[:, None, :]
    re = xr * c - xi * s
    im = xr * s + xi * c
    return torch.stack([re, im], dim=-1).view(L, H, d).float().to(torch.bfloat16)


def norm_rope(x_lin, w, eps, heads, table, grid_hw, start_frame):
    """One projection [L, C] bf16 -> the roped bf16 [L, heads, 128] the attention reads."""
    L = x_lin.shape[0]
    n = rms_norm(x_lin, w, eps, heads).view(L, heads, HEAD_DIM)
    cos, sin = rope_cos_sin(table, L, grid_hw, start_frame)
    return rope_apply(n, cos, sin)
