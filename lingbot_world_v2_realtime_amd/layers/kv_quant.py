"""Pre-quantised chunk memory for the chunk-plus-memory self-attention (the memory-cache surface).

The reference prototyped a cache that keeps K as int8 (frozen mean, per-64-token scales) and V as fp8 next
to the bf16 window, re-quantising it on a chunk's first forward and attending with only Q quantised per call
(experiments/modules/sage_kvq.py:38-111). Here the memory is a ring of chunk slots per layer: each chunk is
quantised once, with its own mean and V scales, when its K/V are written, and attention runs over the
current chunk plus the cached ones in one kernel (the per-chunk mean enters as a logit bias q . mean_c; V's
scales are per 64-key block and the matrix cores apply them, so nothing is rescaled between chunks).

Slot bookkeeping is host integers only (as lingbot/layers/kv_cache.py:1-6 keeps its window positions), so a
forward can be captured in a HIP graph. Two ways to choose what a forward attends to:

- Chunk ring (default): the current chunk plus the `slots` - 1 most recent saved chunks, the first
  `sink_chunks` saved chunks kept for good (a slot-granular version of model_fast_kv_ring.py:28-48's ring).
- The reference's token window (`sink_tokens` / `window_tokens`, or `from_frames`): exactly the tokens
  lingbot/layers/kv_cache.py:23-81 keeps -- a sink of the rollout's first `sink_tokens` tokens plus the most
  recent ones, `window_tokens` in all, evicting by shift, the last `max_attention_size` of them attended.
  Here nothing moves: a chunk stays in its slot and the attention reads the range of it that the window still
  covers (a first token and a key count per chunk, any token of the chunk), so the reference's default
  `--sink_size 6 --local_attn_size 18` with 4-frame chunks of 1508-token frames attends chunk 0, the first 3016
  tokens of chunk 1, the two latest saved chunks and the current chunk (27144 keys in 5 slots), and with
  `--local_attn_size 17` the rolling part starts 1508 tokens into the older of its two chunks.
"""
import torch

from .. import kernels

__all__ = ["QuantKVRing", "alloc_cache", "save_chunk", "attend"]


class QuantKVRing:
    """Quantised K/V ring of `slots` chunk slots for each of `num_layers` layers."""

    def __init__(self, num_layers, batch, heads, chunk_len, slots=4, device="cuda", v_terms=2, sink_chunks=0,
                 sink_tokens=None, window_tokens=None, max_attention_size=None):
        self.window_mode = sink_tokens is not None or window_tokens is not None
        if self.window_mode:
            sink_tokens = sink_tokens or 0
            if window_tokens is not None and window_tokens < sink_tokens + chunk_len:
                # kv_cache.plan would roll a negative number of tokens (the reference's unsupported case)
                raise ValueError("window_tokens must hold the sink plus one chunk")
            if slots is None:
                slots = self.slots_needed(chunk_len, sink_tokens, window_tokens)
        if slots < 2 or slots > kernels.MAX_SEGMENTS:
            raise ValueError(f"slots must be in 2..{kernels.MAX_SEGMENTS}")
        if not 0 <= sink_chunks <= slots - 2:   # at least one rolling slot besides the current one
            raise ValueError(f"sink_chunks must be in 0..slots - 2 = {slots - 2}")
        if self.window_mode and sink_chunks:
            raise ValueError("sink_chunks is for the chunk ring; the token window takes sink_tokens")
        self.cache = kernels.RingCache(num_layers, batch, heads, kernels.pad_to(chunk_len, kernels.K_BLOCK),
                                       slots, device, v_terms)
        self.chunk_len = chunk_len
        self.slots = slots
        self.lens = [0] * slots      # valid tokens in each slot (the same for every layer)
        self.sink_chunks = sink_chunks
        self.sink = []               # chunk ring: slots of the first sink_chunks saved chunks (never evicted)
        self.memory = []             # chunk ring: slots of the other saved chunks, oldest first
        # slot this chunk's K/V are quantised into (token window: chosen at the chunk's first write)
        self.current = None if self.window_mode else 0
        # token window: saved chunks as (slot, stream position, tokens), and the reference buffer's shape as
        # stream[0, head) + stream[end - tail, end) (head = every token while nothing was evicted yet)
        self.sink_tokens, self.window_tokens, self.max_attention_size = sink_tokens, window_tokens, max_attention_size
        self.saved = []
        self.head, self.tail, self.end = 0, 0, 0
        self._ws = {}

    @classmethod
    def from_frames(cls, num_layers, batch, heads, frame_seqlen, chunk_frames=4, sink_size=6, local_attn_size=18,
                    device="cuda", v_terms=2, max_attention_size=None, slots=None):
        """The reference's window in latent frames (lingbot/generate.py:98-99; kv_size = frame_seqlen *
        local_attn_size, sink = sink_size * frame_seqlen: lingbot/pipelines/lingbot_world.py:415,
        transformer.py:219); local_attn_size=-1 keeps every token (then `slots` bounds the rollout)."""
        window = None if local_attn_size == -1 else frame_seqlen * local_attn_size
        return cls(num_layers, batch, heads, frame_seqlen * chunk_frames, slots=slots, device=device,
                   v_terms=v_terms, sink_tokens=sink_size * frame_seqlen, window_tokens=window,
                   max_attention_size=max_attention_size)

    @staticmethod
    def slots_needed(chunk_len, sink_tokens, window_tokens):
        """Slots the token window needs with full chunks: the chunks the sink touches, those the rolling part
        touches (window - sink - one chunk tokens), and the current one."""
        if window_tokens is None:
            raise ValueError("a window without eviction keeps every chunk: give the slot count")
        rolling = window_tokens - sink_tokens - chunk_len
        return -(-sink_tokens // chunk_len) + -(-rolling // chunk_len) + 1

    def _workspace(self, layers, n):
        key = (layers, n)
        if key not in self._ws:
            self._ws[key] = kernels.requant_workspace(layers, self.cache.bh, n, self.cache.device)
        return self._ws[key]

    # ---------------------------------------------------------------- token window planning

    def _plan(self, n):
        """The reference buffer after writing an n-token chunk (kv_cache.plan / evict, kv_cache.py:23-61):
        (head, tail, evicted) with the attended tokens stream[0, head) + stream[end - tail, end) + the chunk."""
        head, tail = self.head, self.tail
        held = head + tail
        if self.window_tokens is not None and n + held > self.window_tokens:
            evicted = n + held - self.window_tokens
            rolled = held - evicted - self.sink_tokens
            if rolled < 0:
                raise ValueError("the rolling window is smaller than a chunk")
            if tail == 0:               # first eviction: the buffer splits into the sink and the rolling part
                head = self.sink_tokens
            return head, rolled, evicted
        return head, tail, 0

    def _ranges(self, n):
        """Attended (slot, first token, tokens) in the reference buffer's order: sink, rolling part, current."""
        head, tail, _ = self._plan(n)
        want = [(0, head), (self.end - tail, self.end)] if tail else [(0, head)]
        out = []
        for lo, hi in want:
            for slot, pos, cn in self.saved:
                a, b = max(lo, pos), min(hi, pos + cn)
                if a < b:
                    out.append((slot, a - pos, b - a))
        if self.current is not None:
            out.append((self.current, 0, n))
        if self.max_attention_size is not None:   # kv_cache.window: the last max_attention_size buffer tokens
            drop = sum(r[2] for r in out) - self.max_attention_size
            while drop > 0:
                s, a, c = out[0]
                if c <= drop:
                    out.pop(0)
                    drop -= c
                else:
                    out[0] = (s, a + drop, c - drop)
                    drop = 0
        merged = []   # a chunk the sink ends in and the rolling part starts in, without a gap: one range
        for r in out:
            if merged and merged[-1][0] == r[0] and merged[-1][1] + merged[-1][2] == r[1]:
                merged[-1] = (r[0], merged[-1][1], merged[-1][2] + r[2])
            else:
                merged.append(r)
        return merged

    def _begin_chunk(self, n):
        """Token window: take a slot for a new n-token chunk -- one holding no token the next window reads."""
        head, tail, _ = self._plan(n)
        keep = set()
        for slot, pos, cn in self.saved:
            if pos < head or (tail and pos + cn > self.end - tail):
                keep.add(slot)
        free = [s for s in range(self.slots) if s not in keep]
        if not free:
            raise RuntimeError(f"{self.slots} slots cannot hold this window: use more slots")
        self.saved = [c for c in self.saved if c[0] in keep]
        self.current = free[0]
        self.lens[self.current] = 0

    # ---------------------------------------------------------------- writes, attention, commit

    def write(self, layer, k, v):
        """Quantise this forward's chunk K/V ([B, L, H, 128] bf16, L <= chunk_len) into the current slot of
        `layer`. Every forward of a chunk calls this; the clean (cache-write) forward is the one that stays."""
        n = k.shape[-3]
        if self.window_mode and self.current is None:
            self._begin_chunk(n)
        kernels.kv_requant(k, v, self.cache, self.current, layer0=layer,
                           workspace=self._workspace(1 if k.dim() == 4 else k.shape[0], n))
        self.lens[self.current] = n

    def write_layers(self, k, v, layer0=0):
        """The same for several layers at once: k, v [layers, B, L, H, 128]."""
        n = k.shape[-3]
        if self.window_mode and self.current is None:
            self._begin_chunk(n)
        kernels.kv_requant(k, v, self.cache, self.current, layer0=layer0,
                           workspace=self._workspace(k.shape[0], n))
        self.lens[self.current] = n

    def write_projected(self, layer, k, v, norm_weight, rope, eps=1e-6, k_out=None):
        """write() from the k projection [B, L, H * 128] instead of the roped K: RMSNorm (norm_weight, eps) and
        the rotary embedding (`rope`, a ChunkRope) are applied on the way in. Returns the roped bf16 K."""
        n = k.shape[1]
        if self.window_mode and self.current is None:
            self._begin_chunk(n)
        out = kernels.norm_rope_kv_requant(k, v, self.cache.heads, norm_weight, eps, rope, self.cache,
                                           self.current, layer=layer, k_out=k_out,
                                           workspace=self._workspace(1, n))
        self.lens[self.current] = n
        return out

    def attended_ranges(self):
        """(slot, first token, tokens) the attention reads, in order."""
        if not self.window_mode:
            return [(s, 0, self.lens[s]) for s in self.sink + self.memory + [self.current]]
        if self.current is None:
            raise RuntimeError("the current chunk has no K/V yet: call write() first")
        return self._ranges(self.lens[self.current])

    def attended(self):
        """(slots, lengths, first tokens) the attention reads, in order: the sink chunks, the other saved chunks
        oldest first, then the current chunk; slot s read over tokens [first, first + length)."""
        ranges = self.attended_ranges()
        return [s for s, _, _ in ranges], [c for _, _, c in ranges], [a for _, a, _ in ranges]

    def attend(self, q, layer, sm_scale=None):
        """Attention of q [B, Lq, H, 128] (bf16 or fp16) over the saved chunks plus the current one of `layer`;
        bf16 out."""
        b, lq, h, _ = q.shape
        slots, lens, firsts = self.attended()
        if any(n == 0 for n in lens):
            raise RuntimeError("the current chunk has no K/V yet: call write() first")
        q8, qs, bias = kernels.quant_q(q, "NHD", self.cache, layer, slots)
        out = q.new_empty(q.shape, dtype=torch.bfloat16)
        return kernels.attn_fwd(q8, qs, bias, b, lq, h, self.cache, layer, slots, lens, out, "NHD", sm_scale,
                                seg_firsts=firsts)

    def attend_projected(self, q, layer, norm_weight, rope, eps=1e-6, sm_scale=None):
        """attend() from the q projection [B, Lq, H * 128]: RMSNorm and the rotary embedding fused into the Q
        quantisation. Returns [B, Lq, H, 128] bf16."""
        b, lq = q.shape[0], q.shape[1]
        h = self.cache.heads
        slots, lens, firsts = self.attended()
        if any(n == 0 for n in lens):
            raise RuntimeError("the current chunk has no K/V yet: call write() first")
        q8, qs, bias, _ = kernels.norm_rope_quant_q(q, h, norm_weight, eps, rope, self.cache, layer, slots)
        out = q.new_empty(b, lq, h, kernels.HEAD_DIM)
        return kernels.attn_fwd(q8, qs, bias, b, lq, h, self.cache, layer, slots, lens, out, "NHD", sm_scale,
                                seg_firsts=firsts)

    def commit(self):
        """The chunk is finished (its clean forward was written).

        Chunk ring: it joins the sink while the sink is not full, else the memory; when every slot is taken the
        oldest non-sink chunk is evicted and its slot takes the next chunk.
        Token window: the reference buffer advances as kv_cache.commit does (kv_cache.py:84-88); the next chunk's
        slot is chosen at its first write, when its length is known."""
        if self.current is None or self.lens[self.current] == 0:
            raise RuntimeError("nothing written to the current slot")
        if self.window_mode:
            n = self.lens[self.current]
            head, tail, evicted = self._plan(n)
            if tail or evicted:
                self.head, self.tail = head, tail + n
            else:
                self.head, self.tail = head + n, 0
            self.saved.append((self.current, self.end, n))
            self.end += n
            self.current = None
            return
        (self.sink if len(self.sink) < self.sink_chunks else self.memory).append(self.current)
        if len(self.sink) + len(self.memory) == self.slots:
            self.current = self.memory.pop(0)
        else:
            used = set(self.sink) | set(self.memory)
            self.current = next(s for s in range(self.slots) if s not in used)
        self.lens[self.current] = 0

    def stream_positions(self):
        """Token window: the stream position of every key the attention reads, in order (for checking)."""
        pos = {slot: p for slot, p, _ in self.saved}
        pos[self.current] = self.end
        out = []
        for slot, a, c in self.attended_ranges():
            out.extend(range(pos[slot] + a, pos[slot] + a + c))
        return out


def alloc_cache(num_layers, batch, heads, chunk_len, slots=4, device="cuda", v_terms=2, sink_chunks=0, **window):
    """A quantised chunk ring (cf. sage_kvq.alloc_cache, experiments/modules/sage_kvq.py:38-48); `window` takes
    sink_tokens / window_tokens / max_attention_size for the reference's token window."""
    return QuantKVRing(num_layers, batch, heads, chunk_len, slots, device, v_terms, sink_chunks, **window)


def save_chunk(ring, layer, k, v):
    """Quantise and keep a finished chunk (cf. sage_kvq.requant_all + write_chunk, sage_kvq.py:78-98)."""
    ring.write(layer, k, v)


def attend(q, ring, layer, sm_scale=None):
    """Attention over the ring (cf. sage_kvq.attend, sage_kvq.py:101-111)."""
    return ring.attend(q, layer, sm_scale)
