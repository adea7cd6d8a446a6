"""The token window of QuantKVRing against a CPU restatement of the reference's KV bookkeeping
(oracle/kv_window.py, following lingbot/layers/kv_cache.py:23-88): over whole rollouts, every forward attends
to the same stream positions, index for index and in the same order. No GPU needed: the ring's slot bookkeeping
is host integers, and the writes here record lengths only."""
import pytest

from lingbot_world_v2_realtime_amd.layers import kv_quant
from oracle import kv_window


def _fake_write(ring, n):
    """What write() records, without the device re-quant."""
    if ring.current is None:
        ring._begin_chunk(n)
    ring.lens[ring.current] = n


def _kernel_positions(ring):
    """Stream positions of the keys the attention call reads, from what it is handed: attended()'s (slot, length,
    first token) per chunk, each range checked against the kernel's contract (inside its slot, at most 8)."""
    slots, lens, firsts = ring.attended()
    assert 1 <= len(slots) <= 8
    pos = {slot: p for slot, p, _ in ring.saved}
    pos[ring.current] = ring.end
    out = []
    for s, n, a in zip(slots, lens, firsts):
        assert n >= 1 and a >= 0 and a + n <= ring.cache.cap
        out.extend(range(pos[s] + a, pos[s] + a + n))
    return out


def _rollout(ring, chunk_lens, passes):
    seen = []
    for n in chunk_lens:
        per = []
        for _ in range(passes):
            _fake_write(ring, n)
            per.append(ring.stream_positions())
            assert _kernel_positions(ring) == per[-1]
        seen.append(per)
        ring.commit()
    return seen


@pytest.mark.parametrize("frame,sink,local,chunk_frames,chunks", [
    (1508, 6, 18, 4, 10),    # the reference's defaults (generate.py:98-99): 27144 keys from chunk 4 on
    (50, 6, 18, 4, 12),
    (50, 4, 16, 4, 10),      # sink of exactly one chunk
    (50, 0, 12, 4, 10),      # no sink
    (37, 3, 11, 2, 14),      # sink of 1.5 chunks, odd frame size
    (1508, 6, 17, 4, 9),     # --local_attn_size 17: the rolling part starts 1508 tokens into a chunk
    (1508, 6, 20, 4, 9),     # --local_attn_size 20: it starts 3016 tokens into one
    (50, 6, 19, 4, 10),
    (37, 5, 14, 3, 12),      # sink and rolling part both end / start mid-chunk
])
def test_window_matches_reference_bookkeeping(frame, sink, local, chunk_frames, chunks):
    ring = kv_quant.QuantKVRing.from_frames(1, 1, 1, frame, chunk_frames, sink, local, device="cpu")
    n = frame * chunk_frames
    got = _rollout(ring, [n] * chunks, passes=5)
    want = kv_window.rollout_positions([n] * chunks, 5, frame * local, frame * sink)
    for i in range(chunks):
        for p in range(5):
            assert got[i][p] == want[i][p].tolist(), (i, p)
    assert ring.slots == kv_quant.QuantKVRing.slots_needed(n, frame * sink, frame * local)


def test_reference_default_window_layout():
    """--sink_size 6 --local_attn_size 18, 4-frame chunks of 1508 tokens: from chunk 4 on the attention reads
    chunk 0 whole, the first 3016 tokens of chunk 1, the two latest saved chunks and the current one, every
    range from a chunk's first token, in 5 slots."""
    ring = kv_quant.QuantKVRing.from_frames(1, 1, 1, 1508, 4, 6, 18, device="cpu")
    assert ring.slots == 5
    for c in range(9):
        _fake_write(ring, 6032)
        slots, lens, firsts = ring.attended()
        assert firsts == [0] * len(slots)
        if c >= 4:
            assert lens == [6032, 3016, 6032, 6032, 6032] and sum(lens) == 27144
            assert len(set(slots)) == 5
        else:
            assert lens == [6032] * (c + 1)
        ring.commit()


def test_window_without_eviction_and_ragged_chunks():
    """local_attn_size = -1 keeps everything (kv_cache.plan's global branch); chunks of different lengths."""
    lens = [100, 64, 300, 17, 250]
    ring = kv_quant.QuantKVRing(1, 1, 1, 300, slots=6, device="cpu", sink_tokens=0, window_tokens=None)
    got = _rollout(ring, lens, passes=2)
    want = kv_window.rollout_positions(lens, 2, 10_000, 0, local_attn_size=-1)
    assert [[p for p in c] for c in got] == [[w.tolist() for w in c] for c in want]
    ring = kv_quant.QuantKVRing(1, 1, 1, 300, slots=5, device="cpu", sink_tokens=120, window_tokens=700)
    lens = [300, 250, 300, 120, 300, 300, 200, 300]
    got = _rollout(ring, lens, passes=3)
    want = kv_window.rollout_positions(lens, 3, 700, 120)
    for i in range(len(lens)):
        assert got[i] == [w.tolist() for w in want[i]], i


def test_windows_read_from_mid_chunk():
    """A rolling part that starts inside a chunk (--local_attn_size 17 with sink 6 at the reference's frame size)
    and a max_attention_size that trims the sink or even the current chunk: every chunk range the attention is
    handed, (slot, length, first token), reads exactly the stream positions the reference's buffer holds."""
    ring = kv_quant.QuantKVRing.from_frames(1, 1, 1, 1508, 4, 6, 17, device="cpu")
    for _ in range(6):
        _fake_write(ring, 6032)
        ring.commit()
    _fake_write(ring, 6032)
    slots, lens, firsts = ring.attended()
    # 25636 keys: chunk 0 whole, chunk 1's first 3016 (the sink), the last 1.75 chunks of the rolling part, current
    assert lens == [6032, 3016, 4524, 6032, 6032] and firsts == [0, 0, 1508, 0, 0] and sum(lens) == 17 * 1508
    cases = [dict(frame=1508, sink=6, local=18, mas=20000, chunks=8),   # trims into the sink's first chunk
             dict(frame=1508, sink=6, local=17, mas=8000, chunks=7),    # only part of one saved chunk stays
             dict(frame=50, sink=6, local=18, mas=150, chunks=9),       # less than the current chunk: trimmed too
             dict(frame=37, sink=3, local=11, mas=200, chunks=10)]
    for c in cases:
        n = 4 * c["frame"]
        ring = kv_quant.QuantKVRing.from_frames(1, 1, 1, c["frame"], 4, c["sink"], c["local"], device="cpu",
                                                max_attention_size=c["mas"])
        got = _rollout(ring, [n] * c["chunks"], passes=2)
        want = kv_window.rollout_positions([n] * c["chunks"], 2, c["frame"] * c["local"], c["frame"] * c["sink"],
                                           max_attention_size=c["mas"])
        for i in range(c["chunks"]):
            assert got[i] == [w.tolist() for w in want[i]], (c, i)
            assert len(got[i][0]) == min(c["mas"], len(want[i][0]))


def test_window_refuses_bad_sizes():
    with pytest.raises(ValueError):   # the rolling part would be negative
        kv_quant.QuantKVRing(1, 1, 1, 200, slots=4, device="cpu", sink_tokens=300, window_tokens=400)
    with pytest.raises(ValueError):
        kv_quant.QuantKVRing(1, 1, 1, 200, slots=4, device="cpu", sink_chunks=1, sink_tokens=100,
                             window_tokens=800)
    ring = kv_quant.QuantKVRing(1, 1, 1, 100, slots=2, device="cpu", sink_tokens=0, window_tokens=None)
    for _ in range(2):
        _fake_write(ring, 100)
        ring.commit()
    with pytest.raises(RuntimeError):   # a window that keeps everything outgrows its slots
        _fake_write(ring, 100)
