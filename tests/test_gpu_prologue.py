"""The fused self-attention prologue on the device (through the C-ABI) against the CPU oracle: the roped Q / K,
the int8 Q and its scales and every field of the re-quantised ring slot bit for bit, the logit bias to fp32
rounding, and the whole chunk (projections in, attention out) within the fp32-SDPA tolerance."""
import pytest
import torch

from conftest import record
from oracle import emu
from oracle import prologue as pro

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS = 1e-6


def _k():
    from lingbot_world_v2_realtime_amd import kernels
    return kernels


def _rope(grid_hw, start):
    from lingbot_world_v2_realtime_amd.layers.prologue import ChunkRope, rope_freqs
    return ChunkRope(rope_freqs(DEV), grid_hw[0], grid_hw[1], start)


def _rows(b, n, heads, seed, scale=1.5):
    g = torch.Generator().manual_seed(seed)
    s = torch.exp(torch.randn(b, n, 1, generator=g) * scale)
    return (torch.randn(b, n, heads * 128, generator=g) * s).to(torch.bfloat16)


def _weight(heads, seed):
    g = torch.Generator().manual_seed(seed)
    return (1 + 0.3 * torch.randn(heads * 128, generator=g)).to(torch.bfloat16)


def _oracle_roped(x, w, heads, grid_hw, start):
    """[B, L, C] -> roped [B, L, H, 128] per batch entry."""
    return torch.stack([pro.norm_rope(x[i], w, EPS, heads, pro.rope_table(), grid_hw, start)
                        for i in range(x.shape[0])])


@pytest.mark.parametrize("b,lq,heads,grid_hw,start", [(1, 1, 1, (3, 4), 0), (1, 100, 2, (5, 4), 3),
                                                      (2, 257, 3, (7, 9), 11), (1, 1508, 12, (29, 52), 20),
                                                      (1, 300, 16, (10, 10), 1)])
def test_norm_rope_quant_q_bit_exact(b, lq, heads, grid_hw, start):
    """Including 16 heads (the 1024-thread variant of the kernel) and a 2-entry batch."""
    k = _k()
    q = _rows(b, lq, heads, lq + heads)
    w = _weight(heads, 7)
    q8, qs, bias, roped = k.norm_rope_quant_q(q.to(DEV), heads, w.to(DEV), EPS, _rope(grid_hw, start),
                                              want_roped=True)
    torch.cuda.synchronize()
    ref = _oracle_roped(q, w, heads, grid_hw, start)
    assert torch.equal(roped.cpu(), ref)
    lp = q8.shape[1]
    for i in range(b):
        r8, rs = emu.quant_q(ref[i])
        assert torch.equal(q8.cpu()[i * heads:(i + 1) * heads], r8)
        assert torch.equal(qs.cpu()[i * heads:(i + 1) * heads], rs)
    assert bias is None and lp % 256 == 0


def test_norm_rope_quant_q_bias_and_unfused_equivalence():
    """With several chunks the kernel also writes q . km_c; and its int8 Q equals lbw_quant_q run on its own roped
    output (the unfused sequence), whose bias it matches to fp32 rounding."""
    k = _k()
    heads, lq, n = 3, 400, 190
    ring = k.RingCache(1, 1, heads, k.pad_to(n, 64), 3, DEV)
    for slot in range(3):
        kk = (torch.randn(1, n, heads, 128) + 2 * torch.randn(1, 1, heads, 128)).to(torch.bfloat16)
        vv = torch.randn(1, n, heads, 128).to(torch.bfloat16)
        k.kv_requant(kk.to(DEV), vv.to(DEV), ring, slot)
    q = _rows(1, lq, heads, 5)
    w = _weight(heads, 9)
    rope = _rope((8, 10), 4)
    q8, qs, bias, roped = k.norm_rope_quant_q(q.to(DEV), heads, w.to(DEV), EPS, rope, ring, 0, [2, 0, 1],
                                              want_roped=True)
    u8, us, ubias = k.quant_q(roped, "NHD", ring, 0, [2, 0, 1])
    torch.cuda.synchronize()
    assert torch.equal(q8, u8) and torch.equal(qs, us)
    torch.testing.assert_close(bias, ubias, rtol=1e-5, atol=1e-5)
    ref = _oracle_roped(q, w, heads, (8, 10), 4)[0]
    for c, slot in enumerate([2, 0, 1]):
        exp = emu.q_bias(ref, ring.km[0, slot].cpu())
        torch.testing.assert_close(bias[c, :, :lq].cpu(), exp, rtol=1e-5, atol=1e-4)
        assert torch.equal(bias[c, :, lq:].cpu(), torch.zeros(heads, bias.shape[2] - lq))


def _check_slot(ring, layer, slot, ref, n):
    nb = (n + 63) // 64
    assert torch.equal(ring.km[layer, slot].cpu(), ref["km"])
    assert torch.equal(ring.v_scale[layer, slot, :, :nb].cpu(), ref["v_scale"])
    assert torch.equal(ring.k_scale[layer, slot, :, :nb].cpu(), ref["k_scale"])
    assert torch.equal(ring.k8[layer, slot, :, :nb * 64].cpu(), ref["k8"])
    assert torch.equal(ring.v8[layer, slot, :, :nb].cpu(), ref["v8"])
    assert torch.equal(ring.v8lo[layer, slot, :, :nb].cpu(), ref["v8lo"])


@pytest.mark.parametrize("n,heads,grid_hw,start", [(1, 1, (2, 2), 0), (63, 2, (3, 7), 2), (65, 3, (4, 4), 9),
                                                   (1508, 12, (29, 52), 0), (200, 16, (5, 8), 6)])
def test_norm_rope_kv_requant_bit_exact(n, heads, grid_hw, start):
    k = _k()
    kk = _rows(1, n, heads, n, scale=0.7) + (3 * torch.randn(1, 1, heads * 128)).to(torch.bfloat16)
    v = (torch.randn(1, n, heads, 128) * 1.7).to(torch.bfloat16)
    w = _weight(heads, 11)
    ring = k.RingCache(2, 1, heads, k.pad_to(n, 64), 2, DEV)
    k_out = k.norm_rope_kv_requant(kk.to(DEV), v.to(DEV), heads, w.to(DEV), EPS, _rope(grid_hw, start), ring, 1,
                                   layer=1)
    # the unfused sequence on the kernel's own roped K gives the same slot
    k.kv_requant(k_out, v.to(DEV), ring, 0, layer0=1)
    torch.cuda.synchronize()
    ref_k = _oracle_roped(kk, w, heads, grid_hw, start)
    assert torch.equal(k_out.cpu(), ref_k)
    ref = emu.requant(ref_k[0], v[0])
    _check_slot(ring, 1, 1, ref, n)
    _check_slot(ring, 1, 0, ref, n)


def test_prologue_eps_zero_ragged():
    """eps = 0 (the ABI takes it) with lengths that end inside a 32-row group: the padding rows must stay exact
    zeros (1 / sqrt(0 + 0) would make them NaN and spread into the Q scale and the chunk's K mean), so the int8 Q,
    its scales, the roped K and every ring field stay bit-exact against the oracle, which pads with zeros."""
    k = _k()
    heads, grid_hw = 2, (5, 7)
    for n in (45, 100):
        x = _rows(1, n, heads, 300 + n)
        w = _weight(heads, 13)
        q8, qs, _, roped = k.norm_rope_quant_q(x.to(DEV), heads, w.to(DEV), 0.0, _rope(grid_hw, 1), want_roped=True)
        v = (torch.randn(1, n, heads, 128) * 1.3).to(torch.bfloat16)
        ring = k.RingCache(1, 1, heads, k.pad_to(n, 64), 1, DEV)
        k_out = k.norm_rope_kv_requant(x.to(DEV), v.to(DEV), heads, w.to(DEV), 0.0, _rope(grid_hw, 1), ring, 0)
        torch.cuda.synchronize()
        ref = torch.stack([pro.norm_rope(x[0], w, 0.0, heads, pro.rope_table(), grid_hw, 1)])
        assert torch.equal(roped.cpu(), ref) and torch.equal(k_out.cpu(), ref)
        r8, rs = emu.quant_q(ref[0])
        assert torch.equal(q8.cpu(), r8) and torch.equal(qs.cpu(), rs)
        _check_slot(ring, 0, 0, emu.requant(ref[0], v[0]), n)
        assert torch.isfinite(ring.km[0, 0]).all()


def _sdpa_gpu_fp32(q, k, v):
    """fp32 softmax attention on the GPU, per head: [L, H, D] -> fp32 [Lq, H, D]."""
    qd, kd, vd = (x.to(DEV).float() for x in (q, k, v))
    out = torch.empty(qd.shape, dtype=torch.float32, device=DEV)
    for hh in range(qd.shape[1]):
        s = torch.matmul(qd[:, hh], kd[:, hh].t()) * (qd.shape[-1] ** -0.5)
        out[:, hh] = torch.matmul(torch.softmax(s, dim=1), vd[:, hh])
    return out


def test_full_chunk_from_projections():
    """Chunk 4 of a rollout of 4-frame chunks (29 x 52 latents a frame, 12 heads, the reference's sink of 6
    frames and window of 18) from its projections: the fused path (causal_self_attention, one call per chunk)
    attends chunk 0, the first 3016 tokens of chunk 1, chunks 2 and 3 and itself (27144 keys). Its ring slot
    equals the oracle's re-quant of the oracle-roped K bit for bit, and its output is within the fp32-SDPA gates
    of attention over the oracle-roped Q / K of exactly those tokens."""
    from lingbot_world_v2_realtime_amd.layers.kv_quant import QuantKVRing
    from lingbot_world_v2_realtime_amd.layers.prologue import ChunkRope, causal_self_attention, rope_freqs
    heads, fl, frames = 12, 1508, 4
    n = fl * frames
    ring = QuantKVRing.from_frames(1, 1, heads, fl, chunk_frames=frames, sink_size=6, local_attn_size=18,
                                   device=DEV)
    table = rope_freqs(DEV)
    wq, wk = _weight(heads, 21), _weight(heads, 22)
    roped_k, vs = [], []
    for c in range(5):
        g = torch.Generator().manual_seed(100 + c)
        q = (torch.randn(1, n, heads * 128, generator=g) * 2).to(torch.bfloat16)
        kk = (torch.randn(1, n, heads * 128, generator=g) * 2 + 3 * torch.randn(1, 1, heads * 128, generator=g)
              ).to(torch.bfloat16)
        v = torch.randn(1, n, heads, 128, generator=g).to(torch.bfloat16)
        rope = ChunkRope.for_chunk(table, (frames, 29, 52), current_start=c * n)
        out = causal_self_attention(ring, 0, q.to(DEV), kk.to(DEV), v.to(DEV), heads, wq.to(DEV), wk.to(DEV), rope,
                                    EPS)
        if c < 4:
            ring.commit()
        roped_k.append(_oracle_roped(kk, wk, heads, (29, 52), c * frames)[0])
        vs.append(v[0])
    torch.cuda.synchronize()
    slots, lens, firsts = ring.attended()
    assert lens == [n, 3016, n, n, n] and firsts == [0] * 5
    _check_slot(ring.cache, 0, slots[-1], emu.requant(roped_k[4], vs[4]), n)
    rq = _oracle_roped(q, wq, heads, (29, 52), 4 * frames)[0]
    used = [(0, n), (1, 3016), (2, n), (3, n), (4, n)]
    kcat = torch.cat([roped_k[i][:m] for i, m in used])
    vcat = torch.cat([vs[i][:m] for i, m in used])
    sd = _sdpa_gpu_fp32(rq, kcat, vcat)
    e = (out[0].float() - sd).abs()
    msg = (f"fused prologue + attention, chunk 4 of the reference window (6032 q x 27144 kv, 12 heads) vs fp32 "
           f"SDPA of the oracle-roped Q/K: max {e.max():.3e} mean {e.mean():.3e}; |out| mean {sd.abs().mean():.3e}")
    record(msg)
    assert e.max() < 2e-2 and e.mean() < 1e-3, msg
