"""The cross-attention kernel (lbw_cross_attn_fwd, bf16 in / out, fp32 accumulation) through the C-ABI against
fp32 softmax attention over the same bf16 inputs: the DiT's shape (6032 queries x 512 context tokens, 12 heads),
ragged query / key counts, per-batch key lengths, and the drop-in flash_attention / cached-context paths."""
import pytest
import torch

from conftest import record

pytestmark = pytest.mark.gpu

DEV = "cuda"
# bf16 P and a bf16 output on top of bf16 inputs: errors relative to the output's scale
MAX_REL = 1.5e-2
MEAN_REL = 2e-3


def _k():
    from lingbot_world_v2_realtime_amd import kernels
    return kernels


def _ref(q, k, v, k_lens=None, sm_scale=None):
    """fp32 softmax attention on the GPU per (batch, head): [B, L, H, D] -> fp32 [B, Lq, H, D]."""
    b, lq, h, d = q.shape
    sm = d ** -0.5 if sm_scale is None else sm_scale
    out = torch.empty(b, lq, h, d, dtype=torch.float32, device=DEV)
    for bi in range(b):
        n = k.shape[1] if k_lens is None else int(k_lens[bi])
        for hh in range(h):
            qf = q[bi, :, hh].float()
            kf = k[bi, :n, hh].float().contiguous()
            vf = v[bi, :n, hh].float().contiguous()
            s = torch.matmul(qf, kf.t()) * sm
            out[bi, :, hh] = torch.matmul(torch.softmax(s, dim=1), vf)
    return out


def _inputs(b, lq, lk, h, seed, kscale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(b, lq, h, 128, device=DEV, generator=g).to(torch.bfloat16)
    k = (torch.randn(b, lk, h, 128, device=DEV, generator=g) * kscale).to(torch.bfloat16)
    v = torch.randn(b, lk, h, 128, device=DEV, generator=g).to(torch.bfloat16)
    return q, k, v


def _check(out, ref, what):
    e = (out.float() - ref).abs()
    scale = ref.abs().mean().item()
    msg = (f"{what}: max {e.max().item():.3e} mean {e.mean().item():.3e} (|ref| mean {scale:.3e}; gates "
           f"{MAX_REL:g} / {MEAN_REL:g} of it)")
    assert e.max().item() <= MAX_REL * ref.abs().max().item() + 1e-3, msg
    assert e.mean().item() <= MEAN_REL * scale + 1e-5, msg
    return msg


def test_cross_attention_dit_shape():
    """The DiT's cross-attention: 6032 queries x 512 context tokens, 12 heads, keys scaled so the softmax is
    peaked (the text context of a trained model is not uniform)."""
    k = _k()
    q, kk, v = _inputs(1, 6032, 512, 12, 0, kscale=2.0)
    ctx = k.CrossContext(kk, v)
    out = k.cross_attn_fwd(q, ctx)
    torch.cuda.synchronize()
    record(_check(out, _ref(q, kk, v), "cross-attention 6032 q x 512 ctx, 12 heads vs fp32"))


@pytest.mark.parametrize("b,lq,lk,h", [(1, 1, 1, 1), (1, 100, 63, 2), (1, 257, 65, 3), (2, 130, 200, 2),
                                       (1, 31, 512, 12)])
def test_cross_attention_ragged(b, lq, lk, h):
    k = _k()
    q, kk, v = _inputs(b, lq, lk, h, lq + lk)
    out = k.cross_attn_fwd(q, k.CrossContext(kk, v))
    torch.cuda.synchronize()
    _check(out, _ref(q, kk, v), f"cross b{b} lq{lq} lk{lk} h{h}")


def test_cross_attention_key_lengths_and_scale():
    """Per-batch key counts (the varlen k_lens of the reference's flash call) and an explicit softmax scale:
    keys past a batch entry's count do not take part."""
    k = _k()
    q, kk, v = _inputs(2, 300, 200, 3, 7)
    lens = [137, 1]
    ctx = k.CrossContext(kk, v)
    out = k.cross_attn_fwd(q, ctx, sm_scale=0.05, k_lens=lens)
    torch.cuda.synchronize()
    _check(out, _ref(q, kk, v, lens, 0.05), "cross with k_lens")
    # garbage past the counts changes nothing
    kk2, v2 = kk.clone(), v.clone()
    kk2[0, 137:] = 100.0
    v2[1, 1:] = -50.0
    out2 = k.cross_attn_fwd(q, k.CrossContext(kk2, v2), sm_scale=0.05, k_lens=lens)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_flash_attention_dropin_and_cache():
    """flash_attention(q, k, v, k_lens) (the cross-attention call) and the cached-context path agree bit for bit;
    a float32 call is cast the way the reference's half() does and returns float32."""
    from lingbot_world_v2_realtime_amd.layers.attention import CrossAttnCache, cross_attention, flash_attention
    q, kk, v = _inputs(1, 500, 512, 12, 3)
    a = flash_attention(q, kk, v)
    cache = CrossAttnCache()
    assert not cache.is_init
    cache.fill(kk, v)
    b = cross_attention(q, cache)
    c = flash_attention(q.float(), kk.float(), v.float())
    torch.cuda.synchronize()
    assert torch.equal(a, b) and c.dtype == torch.float32 and torch.equal(c, a.float())
    _check(a, _ref(q, kk, v), "flash_attention drop-in")
