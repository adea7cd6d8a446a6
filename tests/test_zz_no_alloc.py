"""lbw_attn_fwd_noalloc (the attention entry point that allocates nothing: its split-tile partials live in the
library's fixed per-GPU array) against lbw_attn_fwd with a caller workspace, through the C-ABI: two calls in a row,
the second smaller, each bit-identical to the workspace call. Both shapes cut every query tile into pieces, so
the array carries partials in both calls, and the second call reads none of the first call's leftovers."""
import pytest
import torch

from oracle import emu

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(lq, lk, h, seed, mem_chunks):
    from lingbot_world_v2_realtime_amd import kernels
    from lingbot_world_v2_realtime_amd.layers.kv_quant import QuantKVRing
    q, k, v, mem = emu.make_inputs(lq, lk, h=h, seed=seed, mem_chunks=mem_chunks, chunk_len=lk)
    ring = QuantKVRing(1, 1, h, lk, slots=4, device=DEV)
    for mk, mv in mem:
        ring.write(0, mk.to(DEV), mv.to(DEV))
        ring.commit()
    ring.write(0, k.to(DEV), v.to(DEV))
    slots, lens, firsts = ring.attended()
    q8, qs, bias = kernels.quant_q(q.to(DEV), "NHD", ring.cache, 0, slots)
    return q8, qs, bias, ring, slots, lens, firsts


def test_noalloc_matches_workspace_call_twice():
    from lingbot_world_v2_realtime_amd import _lib, kernels
    gx = _lib.load().lbw_attn_workgroups_per_xcd()
    for lq, lk, h, mem in ((1508, 1508, 6, 0), (300, 200, 2, 2)):
        tiles = kernels.pad_to(lq, kernels.Q_TILE) // kernels.Q_TILE * h
        assert tiles // 8 + 1 < gx             # no XCD has a whole tile per workgroup: every tile is split
        q8, qs, bias, ring, slots, lens, firsts = _case(lq, lk, h, seed=lq + h, mem_chunks=mem)
        want = torch.empty(1, lq, h, 128, dtype=torch.bfloat16, device=DEV)
        got = torch.full_like(want, float("nan"))
        kernels.attn_fwd(q8, qs, bias, 1, lq, h, ring.cache, 0, slots, lens, want, seg_firsts=firsts)
        kernels.attn_fwd(q8, qs, bias, 1, lq, h, ring.cache, 0, slots, lens, got, noalloc=True, seg_firsts=firsts)
        torch.cuda.synchronize()
        print(f"noalloc lq={lq} lk={lk} h={h} chunks={len(slots)}: bit-identical {torch.equal(got, want)}",
              flush=True)
        assert torch.equal(got, want)
