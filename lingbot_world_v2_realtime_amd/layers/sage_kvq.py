"""The pre-quantised KV cache surface of experiments/modules/sage_kvq.py (LINGBOT_ATTN=sage_kvq), with the same
function names and arguments, over the HIP kernels.

The reference keeps quantised K/V in a layer's cache dict next to the bf16 window cache["k"] / cache["v"]
([B, kv_size, H, D], the buffers of lingbot/layers/kv_cache.py), re-quantises the attended slice on a chunk's
first forward (`requant_all`), quantises only the newly written tokens on the others (`write_chunk`), and attends
with only Q quantised per call (`attend`). Here the quantised slice is one slot of a one-layer ring cache
(int8 K - mean per 64-token block, e4m3 V with a power-of-two scale per channel and 32-token half-block, plus the
residual plane; the layout of include/lbw_attn.h),
kept under the dict keys "lbw_ring" and "lbw_ws".

One difference, by design: the reference's write_chunk quantises [floor64(start), end) against the mean and V
scale frozen by the last requant_all, with a 1.5x V margin and a clamp for tokens past it (sage_kvq.py:29-35,
78-90), because its re-quant ran in torch. Here write_chunk re-quantises the whole slice [0, end) with fresh
statistics (the 30-layer re-quant of a 6032-token chunk takes ~0.5 ms on MI355X, one layer ~0.02 ms), so every
token is quantised against its own slice's mean and V scales and nothing saturates.
"""
import torch

from .. import kernels

__all__ = ["alloc_cache", "release", "requant_all", "write_chunk", "attend"]

_KEYS = ("lbw_ring", "lbw_ws")


def alloc_cache(shape, dtype, device):
    """Quantised buffers for one layer's cache dict; `shape` = [B, kv_size, H, D] (sage_kvq.py:38-48). `dtype` is
    the dtype of the window the slice is quantised from: bfloat16 or float16."""
    b, kv_size, h, d = shape
    if d != kernels.HEAD_DIM:
        raise ValueError(f"head dim must be {kernels.HEAD_DIM}, got {d}")
    if dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"the quantised cache is filled from bfloat16 or float16 K/V, got {dtype}")
    ring = kernels.RingCache(1, b, h, kernels.pad_to(kv_size, kernels.K_BLOCK), 1, device)
    return {"lbw_ring": ring, "lbw_ws": kernels.requant_workspace(1, b * h, kv_size, ring.device)}


def release(kv_cache):
    """Drop the quantised buffers of every layer's cache dict (sage_kvq.py:51-54)."""
    for c in kv_cache:
        for key in _KEYS:
            c.pop(key, None)


def requant_all(cache, kv_len, margin=None):
    """Fresh K mean and V scales over the attended slice cache["k"/"v"][:, :kv_len], then quantise all of it
    (sage_kvq.py:93-98). `margin` is accepted for the reference's signature; each V scale here is the power of two
    above its own half-block's amax, so no margin is needed."""
    del margin
    k, v = cache["k"][:, :kv_len], cache["v"][:, :kv_len]
    kernels.kv_requant(k, v, cache["lbw_ring"], 0, workspace=cache["lbw_ws"])


def write_chunk(cache, start, end):
    """Make the quantised slice cover cache["k"/"v"][:, :end] after tokens [start, end) were written
    (sage_kvq.py:78-90): the whole slice is re-quantised (see the module docstring)."""
    if not 0 <= start <= end:
        raise ValueError(f"bad token range [{start}, {end})")
    requant_all(cache, end)


def attend(q, cache, kv_len, sm_scale=None):
    """Attention of q [B, Lq, H, D] (NHD, bf16 or fp16) over the quantised slice's first kv_len tokens, only Q
    quantised here (sage_kvq.py:101-111) -> [B, Lq, H, D] bf16."""
    ring = cache["lbw_ring"]
    if not 1 <= kv_len <= ring.cap:
        raise ValueError(f"kv_len {kv_len} outside the cache (1..{ring.cap})")
    b, lq, h, _ = q.shape
    q8, qs, _ = kernels.quant_q(q, "NHD")
    out = torch.empty_like(q, dtype=torch.bfloat16)
    return kernels.attn_fwd(q8, qs, None, b, lq, h, ring, 0, [0], [kv_len], out, "NHD", sm_scale)
