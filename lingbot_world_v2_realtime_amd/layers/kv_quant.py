"""Pre-quantised chunk memory for the chunk-plus-memory self-attention (the memory-cache surface).

The reference prototyped a cache that keeps K as int8 (frozen mean, per-64-token scales) and V as fp8 next
to the bf16 window, re-quantising it on a chunk's first forward and attending with only Q quantised per call
(experiments/modules/sage_kvq.py:38-111). Here the memory is a ring of chunk slots per layer: each chunk is
quantised once, with its own mean and V scales, when its K/V are written, and attention runs over the
current chunk plus the cached ones in one kernel (the per-chunk mean enters as a logit bias q . mean_c, the
per-chunk V scale as a rescale of the accumulator between chunks).

Slot bookkeeping is host integers only (as lingbot/layers/kv_cache.py:1-6 keeps its window positions), so a
forward can be captured in a HIP graph. With `slots` = 4 the attended keys are the current chunk plus the
three most recent saved chunks (a slot-granular version of model_fast_kv_ring.py:28-48's ring).

The reference's window is a sink of the first tokens plus the most recent ones (kv_cache.py:23-58: eviction
shifts the non-sink part left, the sink stays). `sink_chunks` maps that onto whole chunks: the first
`sink_chunks` chunks committed keep their slots for good, and a full ring evicts its oldest non-sink chunk.
`--sink_size 6` frames of 4-frame chunks is 1.5 chunks: sink_chunks=1 keeps the first chunk, 2 a superset.
"""
from .. import kernels

__all__ = ["QuantKVRing", "alloc_cache", "save_chunk", "attend"]


class QuantKVRing:
    """Quantised K/V ring of `slots` chunk slots for each of `num_layers` layers."""

    def __init__(self, num_layers, batch, heads, chunk_len, slots=4, device="cuda", v_terms=2, sink_chunks=0):
        if slots < 2 or slots > kernels.MAX_SEGMENTS:
            raise ValueError(f"slots must be in 2..{kernels.MAX_SEGMENTS}")
        if not 0 <= sink_chunks <= slots - 2:   # at least one rolling slot besides the current one
            raise ValueError(f"sink_chunks must be in 0..slots - 2 = {slots - 2}")
        self.cache = kernels.RingCache(num_layers, batch, heads, kernels.pad_to(chunk_len, kernels.K_BLOCK),
                                       slots, device, v_terms)
        self.chunk_len = chunk_len
        self.slots = slots
        self.lens = [0] * slots      # valid tokens in each slot (the same for every layer)
        self.sink_chunks = sink_chunks
        self.sink = []               # slots holding the first sink_chunks saved chunks (never evicted)
        self.memory = []             # slots holding the other saved chunks, oldest first
        self.current = 0             # slot this chunk's K/V are quantised into
        self._ws = {}

    def _workspace(self, layers, n):
        key = (layers, n)
        if key not in self._ws:
            self._ws[key] = kernels.requant_workspace(layers, self.cache.bh, n, self.cache.device)
        return self._ws[key]

    def write(self, layer, k, v):
        """Quantise this forward's chunk K/V ([B, L, H, 128] bf16, L <= chunk_len) into the current slot of
        `layer`. Every forward of a chunk calls this; the clean (cache-write) forward is the one that stays."""
        n = k.shape[-3]
        kernels.kv_requant(k, v, self.cache, self.current, layer0=layer,
                           workspace=self._workspace(1 if k.dim() == 4 else k.shape[0], n))
        self.lens[self.current] = n

    def write_layers(self, k, v, layer0=0):
        """The same for several layers at once: k, v [layers, B, L, H, 128]."""
        n = k.shape[-3]
        kernels.kv_requant(k, v, self.cache, self.current, layer0=layer0,
                           workspace=self._workspace(k.shape[0], n))
        self.lens[self.current] = n

    def attended(self):
        """(slots, lengths) the attention reads: the sink chunks, the other saved chunks oldest first, then the
        current chunk."""
        slots = self.sink + self.memory + [self.current]
        return slots, [self.lens[s] for s in slots]

    def attend(self, q, layer, sm_scale=None):
        """Attention of q [B, Lq, H, 128] bf16 over the saved chunks plus the current one of `layer`."""
        b, lq, h, _ = q.shape
        slots, lens = self.attended()
        if any(n == 0 for n in lens):
            raise RuntimeError("the current chunk has no K/V yet: call write() first")
        q8, qs, bias = kernels.quant_q(q, "NHD", self.cache, layer, slots)
        out = q.new_empty(q.shape)
        return kernels.attn_fwd(q8, qs, bias, b, lq, h, self.cache, layer, slots, lens, out, "NHD", sm_scale)

    def commit(self):
        """The chunk is finished (its clean forward was written): it joins the sink while the sink is not full,
        else the memory. When every slot is taken the oldest non-sink chunk is evicted and its slot takes the
        next chunk."""
        if self.lens[self.current] == 0:
            raise RuntimeError("nothing written to the current slot")
        (self.sink if len(self.sink) < self.sink_chunks else self.memory).append(self.current)
        if len(self.sink) + len(self.memory) == self.slots:
            self.current = self.memory.pop(0)
        else:
            used = set(self.sink) | set(self.memory)
            self.current = next(s for s in range(self.slots) if s not in used)
        self.lens[self.current] = 0


def alloc_cache(num_layers, batch, heads, chunk_len, slots=4, device="cuda", v_terms=2, sink_chunks=0):
    """A quantised chunk ring (cf. sage_kvq.alloc_cache, experiments/modules/sage_kvq.py:38-48)."""
    return QuantKVRing(num_layers, batch, heads, chunk_len, slots, device, v_terms, sink_chunks)


def save_chunk(ring, layer, k, v):
    """Quantise and keep a finished chunk (cf. sage_kvq.requant_all + write_chunk, sage_kvq.py:78-98)."""
    ring.write(layer, k, v)


def attend(q, ring, layer, sm_scale=None):
    """Attention over the ring (cf. sage_kvq.attend, sage_kvq.py:101-111)."""
    return ring.attend(q, layer, sm_scale)
