"""Host-side logic without a GPU: the chunk ring's slot bookkeeping, layout/stride decoding, the attention
routing of the drop-in, and that the quantized path refuses CPU tensors instead of computing elsewhere."""
import importlib

import pytest
import torch

from lingbot_world_v2_realtime_amd import kernels
from lingbot_world_v2_realtime_amd.layers import attention as attn_mod
from lingbot_world_v2_realtime_amd.layers import kv_quant


def test_ring_layout_sizes():
    r = kernels.RingCache(layers=3, batch=2, heads=5, cap=192, slots=4, device="cpu")
    assert r.k8.shape == (3, 4, 10, 192, 128) and r.k8.dtype == torch.int8
    assert r.k_scale.shape == (3, 4, 10, 3)
    assert r.km.shape == (3, 4, 10, 128)
    assert r.v8.shape == (3, 4, 10, 3, 128, 64) and r.v8lo.shape == (3, 4, 10, 3, 128, 48)
    assert r.v_scale.shape == (3, 4, 10, 3, 256) and r.v_scale.dtype == torch.uint8
    assert kernels.RingCache(1, 1, 1, 64, 2, "cpu", v_terms=1).v8lo is None
    with pytest.raises(ValueError):
        kernels.RingCache(1, 1, 1, 100, 2, "cpu")
    with pytest.raises(ValueError):
        kernels.RingCache(1, 1, 1, 64, 2, "cpu", v_terms=3)


def test_ring_slot_rotation():
    """Saved chunks oldest first, then the current one; with 4 slots the 4th commit evicts the oldest."""
    ring = kv_quant.QuantKVRing(num_layers=1, batch=1, heads=1, chunk_len=100, slots=4, device="cpu")
    assert ring.cache.cap == 128
    seen = []
    for chunk in range(7):
        ring.lens[ring.current] = 100 - chunk        # what write() records
        slots, lens, firsts = ring.attended()
        assert firsts == [0] * len(slots)
        seen.append((slots, lens))
        assert slots[-1] == ring.current and len(set(slots)) == len(slots)
        ring.commit()
    assert seen[0] == ([0], [100])
    assert seen[1] == ([0, 1], [100, 99])
    assert seen[3][0] == [0, 1, 2, 3]
    assert seen[4][0] == [1, 2, 3, 0]                # chunk 4 reuses chunk 0's slot
    assert seen[6][0] == [3, 0, 1, 2]
    assert seen[6][1] == [97, 96, 95, 94]
    with pytest.raises(RuntimeError):
        ring.commit()                                # nothing written to the new current slot


def test_ring_sink_chunks_stay():
    """sink_chunks=1 (the reference's sink of first frames, kv_cache.py:23-58, at chunk granularity): the first
    chunk keeps its slot for good; a full ring evicts the oldest of the others."""
    ring = kv_quant.QuantKVRing(1, 1, 1, 64, slots=4, device="cpu", sink_chunks=1)
    seen = []
    for chunk in range(8):
        ring.lens[ring.current] = 64 - chunk
        seen.append(ring.attended())
        ring.commit()
    assert seen[0][0] == [0]
    assert seen[3][0] == [0, 1, 2, 3]
    assert seen[4][0] == [0, 2, 3, 1]                # chunk 4 takes chunk 1's slot, chunk 0 stays first
    assert seen[5][0] == [0, 3, 1, 2]
    assert seen[7][0] == [0, 2, 3, 1]
    assert seen[7][1] == [64, 59, 58, 57]            # chunk 0's length, then chunks 5, 6 and the current 7
    two = kv_quant.QuantKVRing(1, 1, 1, 64, slots=4, device="cpu", sink_chunks=2)
    for chunk in range(6):
        two.lens[two.current] = 1
        two.commit()
    assert two.attended()[0][:2] == [0, 1]
    for bad in (-1, 3):
        with pytest.raises(ValueError):
            kv_quant.QuantKVRing(1, 1, 1, 64, slots=4, device="cpu", sink_chunks=bad)


def test_ring_refuses_attend_before_write_and_bad_slots():
    ring = kv_quant.QuantKVRing(1, 1, 1, 64, slots=2, device="cpu")
    with pytest.raises(RuntimeError):
        ring.attend(torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16), 0)
    with pytest.raises(ValueError):
        kv_quant.QuantKVRing(1, 1, 1, 64, slots=9, device="cpu")


def test_dims_nhd_hnd():
    x = torch.empty(2, 7, 3, 128)
    assert kernels._dims(x, "NHD") == (2, 7, 3, 7 * 3 * 128, 3 * 128, 128)
    y = torch.empty(2, 3, 7, 128)
    assert kernels._dims(y, "HND") == (2, 7, 3, 3 * 7 * 128, 128, 7 * 128)
    with pytest.raises(ValueError):
        kernels._dims(x, "NDH")
    with pytest.raises(ValueError):
        kernels._dims(torch.empty(7, 3, 128), "NHD")


def test_quantized_path_refuses_cpu_tensors():
    q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device tensor"):
        attn_mod.sage_attention(q, q, q)
    with pytest.raises(NotImplementedError):
        attn_mod.sage_attention(q, q, q, is_causal=True)


def test_attention_routing(monkeypatch):
    """LINGBOT_ATTN=sage sends plain calls to the quantized kernel and everything else to SDPA."""
    calls = []
    monkeypatch.setattr(attn_mod, "_QUANT", True)
    monkeypatch.setattr(attn_mod, "sage_attention", lambda q, k, v, **kw: calls.append(kw) or q.clone())
    q = torch.randn(1, 16, 2, 128)
    out = attn_mod.attention(q, q, q)
    assert len(calls) == 1 and calls[0]["tensor_layout"] == "NHD" and out.dtype == q.dtype
    ref = torch.nn.functional.scaled_dot_product_attention(*(x.transpose(1, 2).bfloat16() for x in (q, q, q)))
    for kw in (dict(causal=True), dict(k_lens=torch.tensor([16])), dict(dropout_p=0.0, q_lens=torch.tensor([16]))):
        with pytest.warns(UserWarning) if ("k_lens" in kw or "q_lens" in kw) else _no_warn():
            out = attn_mod.attention(q, q, q, **kw)
        assert len(calls) == 1
        if not kw.get("causal"):
            assert torch.equal(out, ref.transpose(1, 2).contiguous())
    monkeypatch.setattr(attn_mod, "_QUANT", False)
    attn_mod.attention(q, q, q)
    assert len(calls) == 1


def test_attention_casts_to_dtype(monkeypatch):
    """As the reference does (lingbot/layers/attention.py:30-35), the quantized route gets q / k / v cast to
    `dtype` (bf16 when None) and the result comes back in q's dtype."""
    seen = []
    monkeypatch.setattr(attn_mod, "_QUANT", True)
    monkeypatch.setattr(attn_mod, "sage_attention", lambda q, k, v, **kw: seen.append((q.dtype, k.dtype, v.dtype))
                        or q.clone())
    q = torch.randn(1, 16, 2, 128)
    assert attn_mod.attention(q, q, q).dtype == torch.float32
    assert attn_mod.attention(q, q, q, dtype=torch.float16).dtype == torch.float32
    assert seen == [(torch.bfloat16,) * 3, (torch.float16,) * 3]


class _no_warn:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


def test_env_switch_read_at_import(monkeypatch):
    monkeypatch.setenv("LINGBOT_ATTN", "sage")
    m = importlib.reload(attn_mod)
    assert m._QUANT
    monkeypatch.setenv("LINGBOT_ATTN", "flash")
    m = importlib.reload(attn_mod)
    assert not m._QUANT
    monkeypatch.delenv("LINGBOT_ATTN")
    importlib.reload(attn_mod)


def test_bench_inputs_and_counts_match_the_tests():
    """bench.py generates the same seeded inputs as the parity tests and counts the same work."""
    import bench
    from oracle import emu
    a = bench.synthetic_inputs(70, 130, h=2, seed=5, mem_chunks=2, chunk_len=64)
    b = emu.make_inputs(70, 130, h=2, seed=5, mem_chunks=2, chunk_len=64)
    for x, y in zip(a[:3], b[:3]):
        assert torch.equal(x, y)
    for (xk, xv), (yk, yv) in zip(a[3], b[3]):
        assert torch.equal(xk, yk) and torch.equal(xv, yv)
    assert bench.attention_ops(6032, 24128) == emu.attention_ops(6032, 24128, 12) == 4.0 * 12 * 6032 * 24128 * 128
    assert bench.requant_bytes(6032) == emu.requant_bytes(6032, 12) == 55_607_760
    # the bytes the three passes move: K twice, V once, both V planes (e4m3, bf6), tables, scales, partial sums --
    # within 2 % of the 30-layer total the FETCH_SIZE / WRITE_SIZE counters read (2.545 GB per call in
    # profiles/hbm_traffic_per_call.md)
    moved = 30 * bench.requant_moved_bytes(6032)
    assert moved == 2_517_302_880 and abs(moved / 2.545e9 - 1) < 2e-2


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_same_device_guard():
    """Wrappers refuse tensors spread over devices (a raw pointer of another device would be dereferenced)."""
    import torch
    from lingbot_world_v2_realtime_amd import kernels
    a = torch.zeros(2)
    b = torch.zeros(2, device="meta")
    kernels._same_device("x", a, None, a)
    with pytest.raises(ValueError):
        kernels._same_device("x", a, b)
