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


def _rollout(ring, chunk_lens, passes):
    seen = []
    for n in chunk_lens:
        per = []
        for _ in range(passes):
            _fake_write(ring, n)
            per.append(ring.stream_positions())
        seen.append(per)
        ring.commit()
    return seen


@pytest.mark.parametrize("frame,sink,local,chunk_frames,chunks", [
    (1508, 6, 18, 4, 10),    # the reference's defaults (generate.py:98-99): 27144 keys from chunk 4 on
    (50, 6, 18, 4, 12),
    (50, 4, 16, 4, 10),      # sink of exactly one chunk
    (50, 0, 12, 4, 10),      # no sink
    (37, 3, 11, 2, 14),      # sink of 1.5 chunks, odd frame size
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
        slots, lens = ring.attended()
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


def test_windows_past_the_kernel_prefix_form():
    """A rolling part that ends inside a chunk, or a max_attention_size that trims the sink, reads a chunk from
    past its first token: the positions still follow the reference, and attend() refuses instead of reading the
    wrong keys."""
    ring = kv_quant.QuantKVRing(1, 1, 1, 200, slots=6, device="cpu", sink_tokens=100, window_tokens=650)
    got = _rollout(ring, [200] * 8, passes=1)
    want = kv_window.rollout_positions([200] * 8, 1, 650, 100)
    assert [c[0] for c in got] == [w[0].tolist() for w in want]
    _fake_write(ring, 200)
    with pytest.raises(NotImplementedError):
        ring.attended()
    ring = kv_quant.QuantKVRing(1, 1, 1, 200, slots=6, device="cpu", sink_tokens=300, window_tokens=1000,
                                max_attention_size=750)
    got = _rollout(ring, [200] * 8, passes=1)
    want = kv_window.rollout_positions([200] * 8, 1, 1000, 300, max_attention_size=750)
    assert [c[0] for c in got] == [w[0].tolist() for w in want]


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
