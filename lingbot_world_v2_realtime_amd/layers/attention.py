"""Attention backends of the DiT, with the quantized MI355X kernels in place of SageAttention 2.2.

Mirrors lingbot/layers/attention.py:1-40. `LINGBOT_ATTN=sage` (read at import time, as the reference does
at :22-24) routes the plain batched self-attention call -- no q_lens / k_lens, no dropout, non-causal, the
only way the causal DiT calls it -- through `sage_attention`: INT8 QK^T and FP8 PV in HIP kernels on gfx950.
The cross-attention's `flash_attention` runs a bf16 flash-attention HIP kernel (lbw_cross_attn_fwd); everything
else goes to the paper's attention semantics (reference/wan/modules/attention.py:132-178), served here by PyTorch
SDPA because flash_attn has no ROCm wheel in this stack.
"""
import os
import warnings

import torch

from .. import kernels

__all__ = ["attention", "flash_attention", "sage_attention", "CrossAttnCache", "cross_attention"]

_QUANT = os.environ.get("LINGBOT_ATTN") in ("sage", "sage_kvq")

# Per-call buffers of the drop-in, kept across calls: (batch, heads, device, stream) -> (ring, re-quant workspace).
# One ring per key, sized for the most keys a call has asked for so far and reused by every call with fewer (the
# DiT's key count grows chunk by chunk up to the window, so earlier sizes are never needed again). Every block the
# attention reads is re-quantised by the call itself, so the ring is allocated uninitialised and never cleared;
# keyed by stream, so calls on different streams never share one.
_DROPIN = {}


def _dropin_buffers(b, h, lk, device):
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (b, h, idx, torch.cuda.current_stream(idx).cuda_stream)
    held = _DROPIN.get(key)
    if held is None or held[0].cap < lk:
        cap = kernels.pad_to(lk, kernels.K_BLOCK)
        _DROPIN.pop(key, None)   # the smaller ring is released before the larger one is taken
        ring = kernels.RingCache(1, b, h, cap, 1, dev, zero=False)
        _DROPIN[key] = (ring, kernels.requant_workspace(1, b * h, cap, dev))
    return _DROPIN[key]


def sage_attention(q, k, v, tensor_layout="NHD", is_causal=False, sm_scale=None):
    """Quantized attention, the call `sageattn(q, k, v, tensor_layout, is_causal, sm_scale)` makes on sm_120
    (per-warp int8 Q, mean-smoothed per-block int8 K, fp8 V; lingbot/layers/attention.py:34-35), here with V's
    power-of-two scales per 64-key block, 32-key half and channel.

    q [B, Lq, H, 128], k/v [B, Lk, H, 128] for "NHD" ([B, H, L, 128] for "HND"), bf16 or fp16 (quantised from
    their own format) on the GPU. Returns bf16 in q's layout. The K mean and V scales are taken over all Lk keys
    (one chunk), so the logits need no per-chunk bias. Raises if liblbw_attn.so is missing: there is no fallback.
    """
    if is_causal:
        raise NotImplementedError("the quantized kernel is non-causal; the DiT never calls it causally")
    for name, t in (("q", q), ("k", k), ("v", v)):
        kernels._require_cuda_16(name, t)
    b, lq, h, *_ = kernels._dims(q, tensor_layout)
    bk, lk, hk, *_ = kernels._dims(k, tensor_layout)
    if (bk, hk) != (b, h) or tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not match")
    if tensor_layout == "HND":
        k, v = k.transpose(1, 2), v.transpose(1, 2)
    ring, ws = _dropin_buffers(b, h, lk, q.device)
    kernels.kv_requant(k, v, ring, 0, workspace=ws)
    q8, qs, _ = kernels.quant_q(q, tensor_layout)
    out = torch.empty_like(q, dtype=torch.bfloat16)
    return kernels.attn_fwd(q8, qs, None, b, lq, h, ring, 0, [0], [lk], out, tensor_layout, sm_scale)


def _paper_attention(q, k, v, q_lens=None, k_lens=None, dropout_p=0., softmax_scale=None, q_scale=None,
                     causal=False, window_size=(-1, -1), deterministic=False, dtype=torch.bfloat16,
                     fa_version=None):
    """The paper's attention when flash_attn is absent: SDPA on [B, L, H, D] inputs
    (reference/wan/modules/attention.py:163-178; padding masks are ignored there too)."""
    if q_lens is not None or k_lens is not None:
        warnings.warn("Padding mask is disabled when using scaled_dot_product_attention. It can have a "
                      "significant impact on performance.")
    if q_scale is not None:
        q = q * q_scale
    qt, kt, vt = (x.transpose(1, 2).to(dtype) for x in (q, k, v))
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=None, is_causal=causal,
                                                           dropout_p=dropout_p, scale=softmax_scale)
    return out.transpose(1, 2).contiguous()


_FLASH_DEFAULTS = {"q_lens": None, "dropout_p": 0., "q_scale": None, "causal": False, "window_size": (-1, -1)}


def flash_attention(q, k, v, k_lens=None, **kw):
    """The paper's FlashAttention call (lingbot/layers/attention.py:16-20 -> reference/wan/modules/attention.py:
    23-129) as the DiT's cross-attention makes it: q [B, Lq, H, 128], k / v [B, Lk, H, 128] on the GPU, optional
    per-batch key counts k_lens; bf16 attention with fp32 accumulation in a HIP kernel (lbw_cross_attn_fwd), out in
    q.dtype. Inputs that are not fp16 / bf16 are cast to `dtype` first, as the reference does; the kernel computes
    in bf16. Calls with arguments the kernel does not take (q_lens, dropout, causal, a window, q_scale) get the
    paper's SDPA form instead."""
    opts = {key: kw.get(key, dflt) for key, dflt in _FLASH_DEFAULTS.items()}
    dtype = kw.get("dtype", torch.bfloat16)
    if any(opts[key] != dflt for key, dflt in _FLASH_DEFAULTS.items() if key != "window_size") or \
            tuple(opts["window_size"]) != (-1, -1) or q.shape[-1] != kernels.HEAD_DIM:
        return _paper_attention(q, k, v, k_lens=k_lens, **kw)
    out_dtype = q.dtype

    def half(x):
        return x if x.dtype in (torch.float16, torch.bfloat16) else x.to(dtype)

    qh, kh, vh = (half(x).to(torch.bfloat16) for x in (q, k, v))
    ctx = kernels.CrossContext(kh, vh)
    out = kernels.cross_attn_fwd(qh, ctx, sm_scale=kw.get("softmax_scale"), k_lens=k_lens)
    return out.to(out_dtype)


class CrossAttnCache:
    """One layer's cross-attention K / V kept across the forwards of a generation, in the kernel's layout (the
    reference's crossattn_cache, lingbot/models/lingbot_world/transformer.py:251-266: filled on the first call,
    read by every later one)."""

    def __init__(self):
        self.ctx = None

    @property
    def is_init(self):
        return self.ctx is not None

    def fill(self, k, v):
        """k, v [B, Lk, H, 128] bf16: the normed context keys and values."""
        self.ctx = kernels.CrossContext(k, v)

    def reset(self):
        self.ctx = None


def cross_attention(q, cache, k_lens=None, softmax_scale=None):
    """q [B, Lq, H, 128] bf16 against the filled CrossAttnCache -> [B, Lq, H, 128] bf16."""
    if cache.ctx is None:
        raise RuntimeError("the cross-attention cache is empty: fill() it with the context's K / V first")
    return kernels.cross_attn_fwd(q, cache.ctx, sm_scale=softmax_scale, k_lens=k_lens)


def attention(q, k, v, q_lens=None, k_lens=None, dropout_p=0., softmax_scale=None, q_scale=None,
              causal=False, window_size=(-1, -1), deterministic=False, dtype=None, fa_version=None):
    """Drop-in for lingbot/layers/attention.py:27-40: same arguments, same routing, q.dtype out. Inputs are cast
    to `dtype` (bf16 by default) as the reference does before its Sage call, and quantised from that format (bf16 or
    fp16). A causal call takes the SDPA route: the quantized kernel is non-causal (the
    reference hands causal to Sage; the DiT never calls it causally)."""
    dtype = torch.bfloat16 if dtype is None else dtype
    if _QUANT and q_lens is None and k_lens is None and dropout_p == 0. and not causal:
        out_dtype = q.dtype
        x = sage_attention(q.to(dtype), k.to(dtype), v.to(dtype), tensor_layout="NHD", is_causal=causal,
                           sm_scale=softmax_scale)
        return x.to(out_dtype)
    return _paper_attention(q, k, v, q_lens=q_lens, k_lens=k_lens, dropout_p=dropout_p,
                            softmax_scale=softmax_scale, q_scale=q_scale, causal=causal,
                            window_size=window_size, deterministic=deterministic, dtype=dtype,
                            fa_version=fa_version)
