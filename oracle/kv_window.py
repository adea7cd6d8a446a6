"""CPU restatement of the reference's self-attention KV window bookkeeping (the oracle for which tokens a
forward attends to; test infrastructure only).

The reference keeps, per layer, a bf16 buffer of `kv_size` = frame_seqlen * local_attn_size tokens holding a sink
(the first sink_size frames of the rollout) plus a rolling window, evicting by shifting the non-sink part left
(lingbot/layers/kv_cache.py:23-88; sizes from lingbot/pipelines/lingbot_world.py:414-418 and the
CausalWanSelfAttention call at lingbot/models/lingbot_world/transformer.py:219-226). This module replays that
state machine on a buffer of *stream positions* (token t of the rollout is the integer t) instead of K/V values,
so what a forward reads is a list of stream positions that a test can compare index for index.
"""
import numpy as np


class PositionWindow:
    """One layer's KV buffer, holding stream positions (-1 = never written)."""

    def __init__(self, kv_size, sink_tokens, local_attn_size=1, max_attention_size=1_000_000):
        # kv_cache.allocate (kv_cache.py:11-20): a [kv_size] buffer and host-int end indices
        self.buf = np.full(kv_size, -1, dtype=np.int64)
        self.kv_size = kv_size
        self.sink_tokens = sink_tokens
        self.local_attn_size = local_attn_size     # -1: no eviction (a global cache)
        self.max_attention_size = max_attention_size
        self.global_end = 0
        self.local_end = 0

    def plan(self, num_new, current_start):
        """kv_cache.plan (kv_cache.py:23-49): (evicted, rolled, local_start, local_end_index, current_end)."""
        current_end = current_start + num_new
        evicted = rolled = 0
        if self.local_attn_size == -1:
            local_end_index, local_start = current_end, current_start
        elif current_end > self.global_end and num_new + self.local_end > self.kv_size:
            evicted = num_new + self.local_end - self.kv_size
            rolled = self.local_end - evicted - self.sink_tokens
            local_end_index = self.local_end + current_end - evicted - self.global_end
            local_start = local_end_index - num_new
        else:
            local_end_index = self.local_end + current_end - self.global_end
            local_start = local_end_index - num_new
        return evicted, rolled, local_start, local_end_index, current_end

    def forward(self, num_new, current_start):
        """One attention call's write + window + commit (transformer.py:219-226): returns the stream positions
        the call attends to, in buffer order."""
        evicted, rolled, s0, e0, current_end = self.plan(num_new, current_start)
        if evicted:
            # kv_cache.evict (kv_cache.py:52-61): non-sink tokens shift left by `evicted`
            s = self.sink_tokens
            if rolled < 0:
                raise ValueError("the rolling window is smaller than a chunk (the reference's unsupported case)")
            self.buf[s:s + rolled] = self.buf[s + evicted:s + evicted + rolled].copy()
        # kv_cache.write (kv_cache.py:64-75)
        self.buf[s0:e0] = np.arange(current_start, current_end)
        # kv_cache.window (kv_cache.py:78-81)
        start = max(0, e0 - self.max_attention_size)
        seen = self.buf[start:e0].copy()
        # kv_cache.commit (kv_cache.py:84-88)
        self.global_end, self.local_end = current_end, e0
        return seen


def rollout_positions(chunk_lens, passes, kv_size, sink_tokens, local_attn_size=1,
                      max_attention_size=1_000_000):
    """Attended stream positions of every forward of a rollout: chunk i (chunk_lens[i] tokens, starting where the
    previous one ended) runs `passes` forwards at the same current_start (the denoising steps and the clean pass,
    lingbot/pipelines/lingbot_world.py:510-553). Returns [[positions of each pass] per chunk]."""
    w = PositionWindow(kv_size, sink_tokens, local_attn_size, max_attention_size)
    out, start = [], 0
    for n in chunk_lens:
        out.append([w.forward(n, start) for _ in range(passes)])
        start += n
    return out
