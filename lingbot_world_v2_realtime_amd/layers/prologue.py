"""The self-attention prologue of a causal DiT block: RMSNorm of the q / k projections and the 3-axis rotary
embedding, fused on the device with the quantisation that consumes them.

The reference computes, per block (lingbot/models/lingbot_world/transformer.py:199-226):
    q = norm_q(Wq x); k = norm_k(Wk x); v = Wv x          WanRMSNorm over all heads * 128 channels
    q, k = causal_rope_apply(q / k, freqs)                 fp64 rotation by the chunk's (frame, h, w) angles
    kvc.write(k, v); out = attention(q, k_window, v_window)
Here the projections go straight into two kernels: one makes the quantised Q (and the per-chunk logit bias), the
other the roped K and the chunk's quantised ring slot, so the roped Q never reaches memory and the roped K is
read back once instead of twice.
"""
from dataclasses import dataclass

import torch

from .. import kernels
from ..kernels import HEAD_DIM

__all__ = ["rope_freqs", "ChunkRope", "norm_rope", "causal_self_attention"]


def _rope_params(rows, dim, theta=10000.0):
    """Complex rotations [rows, dim / 2], angle t * theta^(-2i / dim), as reference/wan/modules/model.py:29-36
    builds them (float64 on the CPU)."""
    inv = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64),
                          torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.outer(torch.arange(rows, dtype=torch.float64), inv)
    return torch.polar(torch.ones_like(ang), ang)


_FREQS = {}


def rope_freqs(device, d=HEAD_DIM, rows=1024):
    """The model's (cos, sin) table, float64 [rows, d / 2, 2]: frame, height and width sections of d - 4 (d // 6),
    2 (d // 6) and 2 (d // 6) channels (transformer.py:553-556). Built once per device."""
    dev = torch.device(device)
    key = (dev, d, rows)
    if key not in _FREQS:
        s = d // 6
        t = torch.view_as_real(torch.cat([_rope_params(rows, d - 4 * s), _rope_params(rows, 2 * s),
                                          _rope_params(rows, 2 * s)], dim=1)).contiguous()
        _FREQS[key] = t.to(dev)
    return _FREQS[key]


@dataclass
class ChunkRope:
    """The rotation of one forward's chunk: the table, the latent grid (h, w) of a frame and the chunk's first
    latent frame (causal_rope_freqs(grid_sizes, freqs, start_frame=current_start // frame_seqlen),
    transformer.py:53-77, 664-665)."""
    table: torch.Tensor
    grid_h: int
    grid_w: int
    start_frame: int

    @classmethod
    def for_chunk(cls, table, grid_size, current_start=0):
        """grid_size: (frames, h, w) of the chunk; current_start: its first token in the rollout."""
        _, h, w = grid_size
        return cls(table, int(h), int(w), int(current_start) // (int(h) * int(w)))


def norm_rope(x, heads, weight, eps, rope):
    """RMSNorm + rotary embedding of one projection [B, L, heads * 128] bf16 -> roped bf16 [B, L, heads, 128]
    (the reference's norm_q + causal_rope_apply), computed by the fused Q kernel."""
    return kernels.norm_rope_quant_q(x, heads, weight, eps, rope, want_roped=True)[3]


def causal_self_attention(ring, layer, q, k, v, heads, norm_q_weight, norm_k_weight, rope, eps=1e-6,
                          sm_scale=None, k_out=None):
    """Self-attention of one chunk from its projections: q, k [B, L, heads * 128], v [B, L, heads, 128] (bf16) ->
    [B, L, heads, 128] bf16, with the chunk's K/V quantised into the ring's current slot of `layer` (the
    transformer.py:199-226 sequence without the linears). `ring` is a QuantKVRing; call ring.commit() after a
    chunk's clean forward, as with ring.write."""
    ring.write_projected(layer, k, v, norm_k_weight, rope, eps, k_out=k_out)
    return ring.attend_projected(q, layer, norm_q_weight, rope, eps, sm_scale)
