"""The rowwise FP8 quantisation's oracle (oracle/fp8.py) pinned on the CPU by what fixes it independently: the
e4m3 grid from the format's definition, exact powers of two, the zero row, the row max landing on 448, and the
round-to-nearest-even error bound."""
import numpy as np
import torch

from oracle import fp8


def e4m3_values():
    """Every finite non-negative e4m3fn value from the format: 4 exponent bits (bias 7), 3 mantissa bits,
    subnormals at exponent 0, S.1111.111 is NaN (so the largest is 1.75 * 2^8 = 448)."""
    vals = []
    for e in range(16):
        for m in range(8):
            if e == 15 and m == 7:
                continue
            vals.append(m / 8 * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
    return np.array(sorted(set(vals)))


def test_values_land_on_the_e4m3_grid_nearest():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(64, 256, generator=g) * torch.exp(torch.randn(64, 1, generator=g) * 3)).to(torch.bfloat16)
    bits, scale = fp8.quant_rows(x)
    grid = e4m3_values()
    y = (x.float() / scale).numpy()
    q = bits.view(torch.float8_e4m3fn).float().numpy()
    assert np.isin(np.abs(q), grid).all()
    # nearest grid point (ties to even mantissa): |y - q| is the smallest distance to the grid
    d = np.abs(np.abs(y)[..., None] - grid[None, None, :]).min(-1)
    assert np.allclose(np.abs(np.abs(y) - np.abs(q)), d, rtol=0, atol=0)
    # every row's max maps to +-448 exactly
    assert (np.abs(q).max(1) == 448.0).all()


def test_exact_scales_and_special_rows():
    x = torch.zeros(3, 32)
    x[1, :] = torch.linspace(-3.5, 3.5, 32)
    x[1, 7] = 448.0 * 2 ** -5            # amax 14 = 448 * 2^-5: the scale is exactly 2^-5
    bits, scale = fp8.quant_rows(x)
    assert scale[0, 0].item() == np.float32(1e-12)         # the floor: a zero row stays zero
    assert torch.equal(bits[0], torch.zeros(32, dtype=torch.uint8))
    assert scale[1, 0].item() == 2.0 ** -5
    # with a power-of-two scale the division is exact: the bits are e4m3(x * 32) itself
    assert torch.equal(bits[1], (x[1] * 32).to(torch.float8_e4m3fn).view(torch.uint8))
    deq = fp8.dequant_rows(bits, scale)
    rel = ((deq[1] - x[1]).abs() / x[1].abs().clamp(min=2.0 ** -9 * 2 ** -5)).max().item()
    assert rel <= 2 ** -4                                 # half a step of a 3-bit mantissa


def test_bf16_and_fp32_inputs_agree_on_bf16_values():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(10, 48, generator=g).to(torch.bfloat16)
    b1, s1 = fp8.quant_rows(x)
    b2, s2 = fp8.quant_rows(x.float())
    assert torch.equal(b1, b2) and torch.equal(s1, s2)


def _ref_mx_formula(x):
    """The reference's MXFP8 quantiser as written (lingbot/layers/linear.py:42-50): the exponent through fp32
    log2 / ceil / exp2."""
    m, k = x.shape
    xb = x.float().view(m, k // 32, 32)
    amax = xb.abs().amax(-1, keepdim=True).clamp(min=2.0 ** -126)
    scale = torch.exp2(torch.ceil(torch.log2(amax / 448)))
    q = (xb / scale).to(torch.float8_e4m3fn).view(m, k)
    return q.view(torch.uint8), scale.view(m, k // 32)


def test_mx_matches_the_reference_formula_away_from_power_of_two_boundaries():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(200, 512, generator=g) * torch.exp(torch.randn(200, 16, 1, generator=g) * 3).repeat_interleave(32, 1).view(200, 512))
    x = x.to(torch.bfloat16)
    bits, e8 = fp8.quant_mx(x)
    rb, rs = _ref_mx_formula(x)
    scale = torch.ldexp(torch.ones(e8.shape), e8.long() - 127)
    assert torch.equal(scale, rs)          # random groups never land within an ulp of a boundary
    assert torch.equal(bits, rb)


def _nan_equal(a, b):
    """e4m3 bytes equal, except that any NaN code (0x7F / 0xFF) matches any other: NaN's sign is not defined."""
    na = (a & 0x7F) == 0x7F
    nb = (b & 0x7F) == 0x7F
    return torch.equal(na, nb) and torch.equal(a[~na], b[~nb])


def _nonfinite_rows(dtype):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(4, 128, generator=g)
    x[0, 5] = float("nan")            # NaN row: everything NaN
    x[1, 70] = float("inf")           # infinite row: +-0, NaN at the infinity
    x[1, 3] = -0.0
    x[2, 0] = -float("inf")
    return x.to(dtype)


def test_rows_nonfinite_follow_the_reference():
    """A row holding a NaN or an infinity: the reference's formula (amax, clamp, divide, cast; linear.py:15-26) makes
    the NaN row all NaN, and the infinite rows' finite values signed zeros with NaN at the infinities. The oracle
    gives the same bytes (up to NaN's sign) and the same scales."""
    for dtype in (torch.bfloat16, torch.float32):
        x = _nonfinite_rows(dtype)
        bits, scale = fp8.quant_rows(x)
        xf = x.float()
        rs = (xf.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12)
        rb = (xf / rs).to(torch.float8_e4m3fn).view(torch.uint8)
        assert _nan_equal(bits, rb)
        assert torch.isnan(scale[0]).all() and torch.isinf(scale[1:3]).all() and torch.isfinite(scale[3]).all()
        assert ((bits[0] & 0x7F) == 0x7F).all()
        assert bits[1, 3] == 0x80 and ((bits[1, 70] & 0x7F) == 0x7F) and ((bits[1] & 0x7F) == 0).sum() == 127


def test_mx_nonfinite_groups_follow_the_reference_formula():
    """Groups holding a NaN or an infinity: the reference's log2 / ceil / exp2 formula gives them a NaN / inf scale,
    whose E8M0 byte is 255, and x / scale (NaN, or +-0 with NaN at the infinity); finite groups of the same rows keep
    their normal scales."""
    x = _nonfinite_rows(torch.bfloat16)
    bits, e8 = fp8.quant_mx(x)
    rb, rs = _ref_mx_formula(x)
    ref_e8 = rs.to(torch.float8_e8m0fnu).view(torch.uint8)
    assert torch.equal(e8, ref_e8)
    assert e8[0, 0] == 255 and e8[1, 2] == 255 and e8[2, 0] == 255 and (e8[3] != 255).all()
    assert _nan_equal(bits, rb)


def test_mx_exact_exponent_at_a_boundary():
    """amax / 448 one ulp above 2^k: the exact ceil is k + 1 (so x / scale stays <= 448); fp32 log2 may round
    onto k. A group whose amax / 448 is exactly 2^k gets scale 2^k and its max maps to 448."""
    x = torch.zeros(2, 32)
    x[0, 0] = 448.0 * 2.0 ** -3                           # q = 2^-3 exactly
    q1 = torch.nextafter(torch.tensor(2.0 ** -3), torch.tensor(1.0))
    x[1, 0] = (q1 * 448).item()
    bits, e8 = fp8.quant_mx(x)
    assert e8[0, 0].item() == 127 - 3 and bits[0, 0].view(torch.float8_e4m3fn).item() == 448.0
    qv = (x[1, 0] / torch.tensor(448.0)).item()
    if qv > 2.0 ** -3:                                      # the product rounded above the power of two
        assert e8[1, 0].item() == 127 - 2
    dq = fp8.dequant_mx(bits, e8)
    assert torch.equal(dq[0], x[0])


def test_gelu_tanh_against_torch_and_identities():
    """The oracle's GELU (tanh form, exact then rounded once to bf16) against torch's own nn.GELU(approximate='tanh')
    evaluated in fp32 on the CPU: for x >= -2 the same bf16 value for every input; below, torch's 1 + tanh(u)
    cancels (its values there are off by up to ~1e-7 absolute and
    reach -0 early), so only the absolute agreement holds -- far below a quantisation step of any row holding
    values of order one. Independent of both formulas: GELU(x) - GELU(-x) = x, GELU(0) = 0, GELU(x) -> x for large
    x and -> -0 for large negative x, and the non-finite cases of the tanh form."""
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(200000, generator=g) * 4).to(torch.bfloat16)
    ours = fp8.gelu_tanh_bf16(x).float()
    theirs = torch.nn.functional.gelu(x.float(), approximate="tanh").to(torch.bfloat16).float()
    step = torch.ldexp(torch.ones_like(ours), (torch.floor(torch.log2(ours.abs().clamp(min=2.0 ** -126))) - 7).int())
    near = x.float() >= -2
    assert torch.equal(ours[near], theirs[near])
    assert ((ours - theirs).abs() <= torch.maximum(step, torch.tensor(1e-6)))[~near].all()
    xd = x.double()
    odd = fp8.gelu_tanh_bf16(x).double() - fp8.gelu_tanh_bf16(-x).double()
    assert ((odd - xd).abs() <= 2.0 ** -7 * xd.abs() + 2.0 ** -120).all()   # two bf16 roundings
    special = torch.tensor([0.0, 30.0, -30.0, float("inf"), -float("inf"), float("nan")]).to(torch.bfloat16)
    r = fp8.gelu_tanh_bf16(special).float()
    assert r[0] == 0 and r[1] == 30.0 and r[2] == 0 and torch.signbit(r[2])
    assert r[3] == float("inf") and r[4].isnan() and r[5].isnan()


def test_mx_grid_zero_groups_and_error_bound():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(16, 256, generator=g)
    x[0, :32] = 0
    bits, e8 = fp8.quant_mx(x)
    assert e8[0, 0].item() == 0 and torch.equal(bits[0, :32], torch.zeros(32, dtype=torch.uint8))   # 2^-127 floor
    q = bits.view(torch.float8_e4m3fn).float()
    grid = e4m3_values()
    assert np.isin(np.abs(q.numpy()), grid).all() and q.abs().max().item() <= 448
    dq = fp8.dequant_mx(bits, e8)
    big = x.abs() > x.abs().view(16, 8, 32).amax(-1).repeat_interleave(32, 1) * 2 ** -5
    assert ((dq - x).abs()[big] <= x.abs()[big] * 2 ** -4).all()
