"""MI355X-native (gfx950) quantized attention for the LingBot-World causal DiT.

The hot path of the reference's self-attention -- per-block INT8 Q/K with K mean-smoothing, INT8 QK^T with
int32 accumulation, an online softmax, FP8-e4m3 PV over a chunk-plus-memory KV cache, and the K/V re-quant
when a finished chunk is saved -- as hand-written HIP kernels in liblbw_attn.so behind the reference's
Python call surface (lingbot/layers/attention.py).
"""
from . import _lib  # noqa: F401
from .layers.attention import attention, flash_attention, sage_attention  # noqa: F401
from .layers import kv_quant, prologue  # noqa: F401

__all__ = ["attention", "flash_attention", "sage_attention", "kv_quant", "prologue"]
