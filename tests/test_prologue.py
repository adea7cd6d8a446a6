"""The self-attention prologue's oracle (RMSNorm + 3-axis rotary embedding, oracle/prologue.py) pinned on the CPU
against what fixes it independently: the rotation table's closed form, the original Wan rope_apply's complex
formulation and its expand/cat indexing, torch's own bf16 casts, and the RMSNorm formula evaluated by torch's
reductions. The device kernels are checked against this oracle bit for bit in the GPU tests."""
import math

import numpy as np
import pytest
import torch

from oracle import prologue as pro
from lingbot_world_v2_realtime_amd.layers import prologue as product


def test_rope_table_closed_form():
    t = pro.rope_table()
    assert t.shape == (1024, 64, 2) and t.dtype == torch.float64
    # sections of 22, 21, 21 pairs; pair i of a section of dim c runs at 10000^(-2i / c)
    dims = [128 - 4 * 21, 42, 42]
    pairs = [c // 2 for c in dims]
    assert pairs == list(pro.rope_sections()) == [22, 21, 21]
    pos = np.arange(1024, dtype=np.float64)[:, None]
    j0 = 0
    for c, npair in zip(dims, pairs):
        ang = pos * (10000.0 ** (-(2 * np.arange(npair)) / c))[None, :]
        np.testing.assert_allclose(t[:, j0:j0 + npair, 0].numpy(), np.cos(ang), rtol=0, atol=2e-13)
        np.testing.assert_allclose(t[:, j0:j0 + npair, 1].numpy(), np.sin(ang), rtol=0, atol=2e-13)
        j0 += npair
    # the package builds the same table bit for bit
    assert torch.equal(product.rope_freqs("cpu"), t)


def _wan_rope_cos_sin(table, f, h, w, start_frame):
    """cos / sin per token by the original Wan rope_apply's construction (reference/wan/modules/model.py:40-67):
    the three section tables expanded over the (f, h, w) grid and concatenated, in complex form."""
    freqs = torch.view_as_complex(table.contiguous())
    c = freqs.shape[1]
    parts = freqs.split([c - 2 * (c // 3), c // 3, c // 3], dim=1)
    fi = torch.cat([
        parts[0][start_frame:start_frame + f].view(f, 1, 1, -1).expand(f, h, w, -1),
        parts[1][:h].view(1, h, 1, -1).expand(f, h, w, -1),
        parts[2][:w].view(1, 1, w, -1).expand(f, h, w, -1)], dim=-1).reshape(f * h * w, -1)
    return fi


@pytest.mark.parametrize("grid,start", [((2, 3, 5), 0), ((3, 4, 2), 7), ((1, 29, 52), 20)])
def test_rope_indexing_matches_wan_grid_expansion(grid, start):
    f, h, w = grid
    t = pro.rope_table()
    cos, sin = pro.rope_cos_sin(t, f * h * w, (h, w), start)
    ref = _wan_rope_cos_sin(t, f, h, w, start)
    assert torch.equal(cos, ref.real) and torch.equal(sin, ref.imag)
    # a chunk that is not a whole number of frames continues the same map
    cos2, _ = pro.rope_cos_sin(t, f * h * w - 3, (h, w), start)
    assert torch.equal(cos2, cos[:-3])


def test_torch_casts_double_to_bf16_through_fp32():
    """The reference's .type_as(x) on the fp64 rotation is torch's double -> bf16 cast, which rounds to fp32
    first; the oracle (and the kernel) round the same way. 1 + 2^-8 + 2^-40 is above the bf16 midpoint
    1 + 2^-8 but rounds to it in fp32, then to even."""
    x = torch.tensor([1 + 2 ** -8 + 2 ** -40, -(1 + 2 ** -8 + 2 ** -40), 1 + 3 * 2 ** -8 - 2 ** -40],
                     dtype=torch.float64)
    assert x.to(torch.bfloat16).tolist() == [1.0, -1.0, 1.015625]
    assert torch.equal(x.to(torch.bfloat16), x.float().to(torch.bfloat16))
    g = torch.Generator().manual_seed(0)
    y = torch.randn(200000, dtype=torch.float64, generator=g) * 3
    assert torch.equal(y.to(torch.bfloat16), y.float().to(torch.bfloat16))


def _rand_rows(L, C, seed):
    g = torch.Generator().manual_seed(seed)
    scale = torch.exp(torch.randn(L, 1, generator=g) * 1.5)             # token norms over ~2 decades
    return (torch.randn(L, C, generator=g) * scale).to(torch.bfloat16)


def test_rope_apply_matches_complex_product():
    """The real-pair rotation equals the complex product of the original rope_apply, cast the same way."""
    L, H = 600, 3
    x = _rand_rows(L, H * 128, 1).view(L, H, 128)
    t = pro.rope_table()
    cos, sin = pro.rope_cos_sin(t, L, (6, 10), 3)
    got = pro.rope_apply(x, cos, sin)
    xc = torch.view_as_complex(x.double().reshape(L, H, 64, 2))
    ref = torch.view_as_real(xc * torch.complex(cos, sin)[:, None, :]).reshape(L, H, 128).to(torch.bfloat16)
    diff = (got.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert diff.max().item() <= 1 and (diff > 0).float().mean().item() < 1e-4
    # position 0 of frame 0 is the identity; rotations keep pair norms (up to the bf16 casts)
    c0, s0 = pro.rope_cos_sin(t, 1, (6, 10), 0)
    assert torch.equal(pro.rope_apply(x[:1], c0, s0), x[:1])
    n_in = x.double().view(L, H, 64, 2).norm(dim=-1)
    n_out = got.double().view(L, H, 64, 2).norm(dim=-1)
    assert torch.allclose(n_out, n_in, rtol=2 ** -7, atol=1e-30)


def _torch_rms_norm(x, w, eps):
    """WanRMSNorm.forward (reference/wan/modules/model.py:78-86) evaluated by torch's own fp32 reductions."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)).to(torch.bfloat16) * w


@pytest.mark.parametrize("heads", [1, 3, 12])
def test_rms_norm_matches_torch_formula(heads):
    """The fixed-order fp64 sum and fp64 reciprocal square root differ from torch's fp32 evaluation rarely, by one
    bf16 step before the weight and two after it."""
    C = heads * 128
    x = _rand_rows(2000, C, heads)
    g = torch.Generator().manual_seed(99)
    w = (1 + 0.3 * torch.randn(C, generator=g)).to(torch.bfloat16)
    ones = torch.ones(C, dtype=torch.bfloat16)
    for weight, steps in ((ones, 1), (w, 2)):   # a one-step flip of bf16(x r), times w, can round two steps apart
        got = pro.rms_norm(x, weight, 1e-6, heads)
        ref = _torch_rms_norm(x, weight, 1e-6)
        diff = (got.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
        assert diff.max().item() <= steps and (diff > 0).float().mean().item() < 2e-3
    # the row scale itself: against an fp64 evaluation of 1 / sqrt(mean(x^2) + eps), within an fp32 ulp
    xd = x.double()
    r_exact = 1.0 / torch.sqrt(xd.pow(2).mean(-1) + 1e-6)
    y = pro.rms_norm(x, torch.ones(C, dtype=torch.bfloat16), 1e-6, heads).double()
    ratio = (y.abs().sum(-1) / (xd.abs().sum(-1) * r_exact))
    assert torch.allclose(ratio, torch.ones_like(ratio), rtol=2 ** -7)


def test_rms_norm_special_rows():
    C = 256
    x = torch.zeros(3, C, dtype=torch.bfloat16)
    x[1] = 3.0                                        # constant row: mean(x^2) = 9, r = 1 / sqrt(9 + eps)
    x[2, 5] = -2.0                                    # one nonzero: |y| = sqrt(C) * 2 / sqrt(4 + C eps)
    w = torch.ones(C, dtype=torch.bfloat16)
    y = pro.rms_norm(x, w, 1e-6, 2).float()
    assert torch.equal(y[0], torch.zeros(C))          # an all-zero row stays zero (r = 1 / sqrt(eps))
    assert torch.equal(y[1], torch.full((C,), 1.0))   # 3 / sqrt(9 + 1e-6) rounds to 1 in bf16
    expect = torch.tensor(-2.0 * math.sqrt(C) / math.sqrt(4 + C * 1e-6)).to(torch.bfloat16).float()
    assert y[2, 5] == expect and int((y[2] != 0).sum()) == 1


def test_norm_rope_composes_and_sum_order_is_exact_for_typical_rows():
    """norm_rope is rms_norm then rope_apply; for rows of bf16 values within 2^20 of each other the fp64 sum of
    squares is exact, so the fixed order equals an exact (order-free) evaluation."""
    L, H = 300, 2
    x = _rand_rows(L, H * 128, 5)
    w = (1 + 0.2 * torch.randn(H * 128, generator=torch.Generator().manual_seed(3))).to(torch.bfloat16)
    t = pro.rope_table()
    out = pro.norm_rope(x, w, 1e-6, H, t, (4, 5), 2)
    cos, sin = pro.rope_cos_sin(t, L, (4, 5), 2)
    assert torch.equal(out, pro.rope_apply(pro.rms_norm(x, w, 1e-6, H).view(L, H, 128), cos, sin))
    sq = x.double().pow(2)
    exact = torch.tensor([math.fsum(r) for r in sq.tolist()], dtype=torch.float64)
    seq = sq.view(L, H, 16, 8)
    a = torch.zeros(L, H, 16, dtype=torch.float64)
    for e in range(8):
        a = a + seq[..., e]
    while a.shape[-1] > 1:
        a = a[..., 0::2] + a[..., 1::2]
    tot = torch.zeros(L, dtype=torch.float64)
    for h in range(H):
        tot = tot + a[:, h, 0]
    assert torch.equal(tot, exact)


def test_chunk_rope_start_frame():
    t = product.rope_freqs("cpu")
    r = product.ChunkRope.for_chunk(t, (4, 29, 52), current_start=5 * 1508)
    assert (r.grid_h, r.grid_w, r.start_frame) == (29, 52, 5)
