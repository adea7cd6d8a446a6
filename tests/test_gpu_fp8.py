"""The FP8 linear path on the device: the rowwise e4m3 quantisation kernel (lbw_quant_rows_fp8, through the
C-ABI) bit for bit against the oracle, and FP8Linear (that kernel + hipBLASLt's rowwise-scaled FP8 GEMM) against
the fp32 product of the same quantised operands."""
import pytest
import torch

from conftest import record
from oracle import fp8

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _k():
    from lingbot_world_v2_realtime_amd import kernels
    return kernels


@pytest.mark.parametrize("rows,cols,dtype", [(1, 16, torch.bfloat16), (37, 1536, torch.bfloat16),
                                             (6032, 1536, torch.bfloat16), (100, 8960, torch.bfloat16),
                                             (1536, 1536, torch.float32), (3, 2064, torch.float32),
                                             (9, 4112, torch.bfloat16), (2048, 4096, torch.bfloat16),
                                             (2049, 16, torch.bfloat16), (2050, 2064, torch.float32),
                                             (3000, 1024, torch.float32), (20, 12288, torch.float32),
                                             (64, 16400, torch.bfloat16)])
def test_quant_rows_bit_exact(rows, cols, dtype):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * torch.exp(torch.randn(rows, 1, generator=g) * 2)).to(dtype)
    x[0, :] = 0                                            # the scale floor
    x8, sc = _k().quant_rows_fp8(x.to(DEV))
    torch.cuda.synchronize()
    rb, rs = fp8.quant_rows(x)
    assert torch.equal(x8.view(torch.uint8).cpu(), rb)
    assert torch.equal(sc.cpu(), rs)


def test_quant_rows_signed_zero_and_subnormal_edge():
    """Signed zeros keep their sign and quotients around e4m3's smallest subnormals (2^-9, ties at odd multiples of
    2^-10) round as the reference's division does: row amax 448 makes the scale exactly 1."""
    edge = [0.0, -0.0, 2 ** -10, -2 ** -10, 1.5 * 2 ** -10, 2 ** -9, 3 * 2 ** -10, 2 ** -11, 2 ** -6, 448.0, -448.0,
            0.3, -1e-30, 1e-30, 5 * 2 ** -10, -7 * 2 ** -10]
    for dtype in (torch.bfloat16, torch.float32):
        x = torch.tensor(edge * 2, dtype=torch.float32).reshape(2, -1).to(dtype)
        x[1] *= 3.0 ** 0.5                                   # a scale that is not a power of two
        x8, sc = _k().quant_rows_fp8(x.to(DEV))
        torch.cuda.synchronize()
        rb, rs = fp8.quant_rows(x)
        assert torch.equal(x8.view(torch.uint8).cpu(), rb) and torch.equal(sc.cpu(), rs), dtype
        assert int(rb[0, 1]) == 0x80                          # -0 stays -0


def test_quant_rows_strided_view():
    x = torch.randn(50, 2 * 256, dtype=torch.bfloat16)
    view = x[:, :256]                                      # row stride 512
    x8, sc = _k().quant_rows_fp8(x.to(DEV)[:, :256])
    torch.cuda.synchronize()
    rb, rs = fp8.quant_rows(view)
    assert torch.equal(x8.view(torch.uint8).cpu(), rb) and torch.equal(sc.cpu(), rs)


@pytest.mark.parametrize("m,k,n,bias", [(6032, 1536, 1536, True), (333, 1536, 8960, False), (64, 8960, 1536, True)])
def test_fp8_linear(m, k, n, bias):
    from lingbot_world_v2_realtime_amd.layers.linear import FP8Linear
    g = torch.Generator().manual_seed(m)
    lin = torch.nn.Linear(k, n, bias=bias).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
        if bias:
            lin.bias.copy_(torch.randn(n, generator=g) * 0.1)
    lin = lin.to(DEV)
    f = FP8Linear(lin)
    # a 3-d activation [2, m / 2, k] when m is even (the DiT's [B, L, C]), else 2-d
    shape = (2, m // 2, k) if m % 2 == 0 else (m, k)
    x = torch.randn(*shape, generator=g).to(torch.bfloat16)
    y = f(x.to(DEV))
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and y.shape == (*x.shape[:-1], n)
    # the same quantised operands in fp32 on the CPU
    xb, xs = fp8.quant_rows(x.reshape(-1, k))
    wb, ws = fp8.quant_rows(lin.weight.detach().cpu())
    ref = fp8.dequant_rows(xb, xs) @ fp8.dequant_rows(wb, ws).t()
    if bias:
        ref = ref + lin.bias.detach().cpu().to(torch.bfloat16).float()
    e = (y.reshape(-1, n).float().cpu() - ref).abs()
    scale = ref.abs().max().item()
    assert e.max().item() <= 1e-2 * scale, (e.max().item(), scale)   # bf16 output + fp32 accumulation order
    # and against the bf16 linear it replaces: the fp8 rounding of both operands
    full = (x.reshape(-1, k).float() @ lin.weight.detach().cpu().float().t())
    if bias:
        full = full + lin.bias.detach().cpu().float()
    rel = ((y.reshape(-1, n).float().cpu() - full).norm() / full.norm()).item()
    record(f"FP8Linear {m}x{k}x{n}: vs same-operand fp32 max {e.max().item():.2e} (|ref| max {scale:.2e}); "
           f"vs bf16 linear rel-L2 {rel:.2e}")
    assert rel < 6e-2


def test_fp8_linear_tuned_table():
    """The tuned-solution table (layers/fp8_gemm_solutions.csv) is accepted on this GPU and library version, and
    the shape it covers, the feed-forward down projection 6032 x 8960 -> 1536 with its bias, gives the same-operand
    fp32 result to the tolerance of the default solution."""
    import torch.cuda.tunable as tunable
    from lingbot_world_v2_realtime_amd.layers.linear import FP8Linear, use_tuned_gemms
    m, k, n = 6032, 8960, 1536
    g = torch.Generator().manual_seed(7)
    lin = torch.nn.Linear(k, n).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
        lin.bias.copy_(torch.randn(n, generator=g) * 0.1)
    lin = lin.to(DEV)
    f = FP8Linear(lin)
    x = torch.randn(1, m, k, generator=g).to(torch.bfloat16)
    y0 = f(x.to(DEV))
    try:
        assert use_tuned_gemms()
        y = f(x.to(DEV))
        torch.cuda.synchronize()
    finally:
        tunable.enable(False)
    xb, xs = fp8.quant_rows(x.reshape(-1, k))
    wb, ws = fp8.quant_rows(lin.weight.detach().cpu())
    ref = fp8.dequant_rows(xb, xs) @ fp8.dequant_rows(wb, ws).t() + lin.bias.detach().cpu().to(torch.bfloat16).float()
    scale = ref.abs().max().item()
    e = (y.reshape(-1, n).float().cpu() - ref).abs().max().item()
    e0 = (y0.reshape(-1, n).float().cpu() - ref).abs().max().item()
    record(f"FP8Linear {m}x{k}x{n} with the tuned solution: vs same-operand fp32 max {e:.2e} (default solution "
           f"{e0:.2e}; |ref| max {scale:.2e})")
    assert e <= 1e-2 * scale


def test_convert_to_fp8_selection():
    from lingbot_world_v2_realtime_amd.layers.linear import FP8Linear, convert_to_fp8
    blk = torch.nn.Sequential(torch.nn.Linear(1536, 1536), torch.nn.Sequential(torch.nn.Linear(1536, 8960)),
                              torch.nn.Linear(256, 1536), torch.nn.Linear(1536, 1000)).to(torch.bfloat16).to(DEV)
    n_fp8, n_all = convert_to_fp8(blk)
    assert (n_fp8, n_all) == (2, 4)
    assert isinstance(blk[0], FP8Linear) and isinstance(blk[1][0], FP8Linear)
    assert isinstance(blk[2], torch.nn.Linear) and isinstance(blk[3], torch.nn.Linear)


@pytest.mark.parametrize("rows,rows_pad,cols,dtype", [(1, 128, 32, torch.bfloat16), (100, 128, 1536, torch.bfloat16),
                                                      (6032, 6144, 1536, torch.bfloat16),
                                                      (300, 384, 8960, torch.float32)])
def test_quant_mx_bit_exact(rows, rows_pad, cols, dtype):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * torch.exp(torch.randn(rows, 1, generator=g) * 3)).to(dtype)
    x[0, :64] = 0
    x8, e8 = _k().quant_mx_fp8(x.to(DEV), rows_pad)
    torch.cuda.synchronize()
    rb, re = fp8.quant_mx(x)
    assert torch.equal(x8.view(torch.uint8)[:rows].cpu(), rb)
    assert torch.equal(e8.view(torch.uint8)[:rows].cpu(), re)
    assert not x8.view(torch.uint8)[rows:].any() and (e8.view(torch.uint8)[rows:] == 127).all()


@pytest.mark.parametrize("m,k,n,bias", [(6032, 1536, 1536, True), (100, 1536, 8960, False)])
def test_mxfp8_linear(m, k, n, bias):
    from lingbot_world_v2_realtime_amd.layers.linear import MXFP8Linear
    g = torch.Generator().manual_seed(m + 1)
    lin = torch.nn.Linear(k, n, bias=bias).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
        if bias:
            lin.bias.copy_(torch.randn(n, generator=g) * 0.1)
    f = MXFP8Linear(lin.to(DEV))
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    y = f(x.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    xb, xe = fp8.quant_mx(x)
    wb, we = fp8.quant_mx(lin.weight.detach().cpu())
    ref = fp8.dequant_mx(xb, xe) @ fp8.dequant_mx(wb, we).t()
    if bias:
        ref = ref + lin.bias.detach().cpu().float()
    e = (y.float().cpu() - ref).abs()
    record(f"MXFP8Linear {m}x{k}x{n}: vs same-operand fp32 max {e.max().item():.2e} (|ref| max {ref.abs().max().item():.2e})")
    assert e.max().item() <= 1e-2 * ref.abs().max().item()


def _nan_equal(a, b):
    na, nb = (a & 0x7F) == 0x7F, (b & 0x7F) == 0x7F   # any NaN code matches any other (NaN's sign is not defined)
    return torch.equal(na, nb) and torch.equal(a[~na], b[~nb])


def test_quant_nonfinite_rows():
    """Rows holding a NaN or an infinity, rowwise and MX, against the oracle (which follows the reference's torch
    formulas): a NaN spreads over its row (its group for MX), an infinity makes the row's (group's) finite values
    signed zeros and itself NaN, with scale NaN / inf (E8M0 byte 255); the finite rows are untouched."""
    g = torch.Generator().manual_seed(8)
    for dtype in (torch.bfloat16, torch.float32):
        x = torch.randn(6, 1536, generator=g)
        x[1, 700] = float("nan")
        x[2, 3] = float("inf")
        x[2, 4] = -0.0
        x[4, 1535] = -float("inf")
        x = x.to(dtype)
        x8, sc = _k().quant_rows_fp8(x.to(DEV))
        m8, me = _k().quant_mx_fp8(x.to(DEV), 128)
        torch.cuda.synchronize()
        rb, rs = fp8.quant_rows(x)
        assert _nan_equal(x8.view(torch.uint8).cpu(), rb)
        assert torch.equal(sc.cpu().isnan(), rs.isnan()) and torch.equal(sc.cpu()[~rs.isnan()], rs[~rs.isnan()])
        mb, mer = fp8.quant_mx(x)
        assert _nan_equal(m8.view(torch.uint8)[:6].cpu(), mb)
        assert torch.equal(me.view(torch.uint8)[:6].cpu(), mer)
        assert int(x8.view(torch.uint8)[2, 4].cpu()) == 0x80 and (mer[2, 0] == 255) and (mer[2, 1:] != 255).all()
        # the same rows among 2048 others: the one-wave-per-row kernel of calls with many rows
        big = torch.cat([x, torch.randn(2048, 1536, generator=g).to(dtype)])
        b8, bs = _k().quant_rows_fp8(big.to(DEV))
        torch.cuda.synchronize()
        rb, rs = fp8.quant_rows(big)
        assert _nan_equal(b8.view(torch.uint8).cpu(), rb)
        assert torch.equal(bs.cpu().isnan(), rs.isnan()) and torch.equal(bs.cpu()[~rs.isnan()], rs[~rs.isnan()])


def test_mxfp8_linear_k_not_a_multiple_of_128():
    """in_features 1056 (33 scale groups): the weights and activations are padded with zero columns to 1152 for
    the GEMM's 128-wide scale tile, which leaves the product unchanged: against fp32 of the unpadded MX operands."""
    from lingbot_world_v2_realtime_amd.layers.linear import MXFP8Linear
    g = torch.Generator().manual_seed(9)
    m, k, n = 100, 1056, 1536
    lin = torch.nn.Linear(k, n, bias=True).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
        lin.bias.copy_(torch.randn(n, generator=g) * 0.1)
    f = MXFP8Linear(lin.to(DEV))
    assert f.w8.shape == (1536, 1152) and f.k_pad == 96
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    y = f(x.to(DEV))
    torch.cuda.synchronize()
    xb, xe = fp8.quant_mx(x)
    wb, we = fp8.quant_mx(lin.weight.detach().cpu())
    ref = fp8.dequant_mx(xb, xe) @ fp8.dequant_mx(wb, we).t() + lin.bias.detach().cpu().float()
    e = (y.float().cpu() - ref).abs()
    record(f"MXFP8Linear {m}x{k}x{n} (K padded to 1152): vs same-operand fp32 max {e.max().item():.2e} "
           f"(|ref| max {ref.abs().max().item():.2e})")
    assert e.max().item() <= 1e-2 * ref.abs().max().item()


def test_convert_to_fp8_mx_selection():
    from lingbot_world_v2_realtime_amd.layers.linear import MXFP8Linear, convert_to_fp8
    blk = torch.nn.Sequential(torch.nn.Linear(1536, 1536), torch.nn.Linear(1040, 1536)).to(torch.bfloat16).to(DEV)
    assert convert_to_fp8(blk, mx=True) == (1, 2)   # 1040 is a multiple of 16, not of 32
    assert isinstance(blk[0], MXFP8Linear) and isinstance(blk[1], torch.nn.Linear)


def _e4m3_step(v):
    """Spacing of e4m3 around |v| (fp32 tensor): 2^(e - 3) in the normal range, 2^-9 below it."""
    e = torch.floor(torch.log2(v.abs().clamp(min=2.0 ** -6)))
    return torch.ldexp(torch.ones_like(v), (e - 3).int())


@pytest.mark.parametrize("rows,cols", [(333, 1536), (2048, 1536), (64, 8960), (6, 20000), (3, 16)])
def test_quant_rows_gelu_vs_oracle(rows, cols):
    """GELU (tanh form, bf16) fused into the rowwise quantisation, every kernel form (one wave per row, a workgroup
    per row with the row in registers, rows read twice), against the oracle: the exact GELU rounded once to bf16,
    then the oracle's rowwise quantisation. The kernel's GELU is within a few fp32 ulps of exact, so its bf16 value
    differs from the oracle's only next to a rounding boundary: the scales agree to a bf16 ulp, nearly every code is
    identical, and no dequantised value is more than one e4m3 step away."""
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = (torch.randn(rows, cols, generator=g) * 3).to(torch.bfloat16)
    x[0, :8] = torch.tensor([0.0, -0.0, 10.0, -10.0, -100.0, 100.0, 1e-3, -1e-3]).to(torch.bfloat16)
    x8, sc = _k().quant_rows_fp8_gelu(x.to(DEV))
    torch.cuda.synchronize()
    gx = fp8.gelu_tanh_bf16(x)
    rb, rs = fp8.quant_rows(gx)
    sc = sc.cpu()
    assert ((sc - rs).abs() <= 2.0 ** -8 * rs).all()
    codes = x8.view(torch.uint8).cpu()
    same = (codes == rb).float().mean().item()
    got, want = fp8.dequant_rows(codes, sc), fp8.dequant_rows(rb, rs)
    gap = (got - want).abs()
    step = torch.maximum(_e4m3_step(codes.view(torch.float8_e4m3fn).float()) * sc,
                         _e4m3_step(rb.view(torch.float8_e4m3fn).float()) * rs)
    record(f"quant_rows_gelu {rows}x{cols}: identical codes {same:.5f}, max dequant gap / step "
           f"{(gap / step).max().item():.3f}")
    assert same >= 0.99
    assert (gap <= 1.1 * step).all()
    # the pinned points: GELU(0) = +-0 stays a zero code, GELU(10) = 10, GELU(-100) = -0
    assert int(codes[0, 0]) in (0, 0x80) and int(codes[0, 4]) in (0, 0x80)
    assert abs(float(got[0, 2]) - 10.0) <= float(_e4m3_step(torch.tensor(10.0)) * sc[0])


def test_quant_rows_gelu_nonfinite_and_torch_gelu():
    """Non-finite inputs as the tanh form gives them (+inf -> inf: the row's scale inf; -inf -> NaN and NaN -> NaN:
    the row NaN), finite rows untouched; and on finite rows the fused pass against torch's own GELU on the device
    followed by the unfused quantiser (the two-launch path it replaces)."""
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(2054, 1536, generator=g) * 2).to(torch.bfloat16)
    x[1, 5], x[2, 6], x[3, 7] = float("inf"), -float("inf"), float("nan")
    x8, sc = _k().quant_rows_fp8_gelu(x.to(DEV))
    y = torch.nn.functional.gelu(x.to(DEV), approximate="tanh")
    u8, us = _k().quant_rows_fp8(y)
    torch.cuda.synchronize()
    sc, us = sc.cpu(), us.cpu()
    assert float(sc[1]) == float("inf") and bool(sc[2].isnan()) and bool(sc[3].isnan())
    rb, rs = fp8.quant_rows(fp8.gelu_tanh_bf16(x))
    assert _nan_equal(x8.view(torch.uint8)[1:4].cpu(), rb[1:4])
    fin = torch.ones(x.shape[0], dtype=torch.bool)
    fin[1:4] = False
    assert ((sc[fin] - us[fin]).abs() <= 2.0 ** -8 * us[fin]).all()
    same = (x8.view(torch.uint8).cpu()[fin] == u8.view(torch.uint8).cpu()[fin]).float().mean().item()
    record(f"quant_rows_gelu vs torch gelu + quant_rows: identical codes {same:.5f}")
    assert same >= 0.99


def test_fp8_linear_fused_gelu_and_convert():
    """The DiT feed-forward block with fuse_gelu: convert_to_fp8 turns its GELU into nn.Identity and lets the second
    linear apply it in its activation quantisation; the block's output matches the unfused FP8 block (torch's GELU,
    then the separate quantisation) to the FP8 linears' own tolerance."""
    from lingbot_world_v2_realtime_amd.layers.linear import FP8Linear, convert_to_fp8
    g = torch.Generator().manual_seed(17)

    def ffn():
        torch.manual_seed(3)
        f = torch.nn.Sequential(torch.nn.Linear(1536, 8960), torch.nn.GELU(approximate="tanh"),
                                torch.nn.Linear(8960, 1536), torch.nn.GELU(), torch.nn.Linear(1536, 1536))
        for m in f:
            if isinstance(m, torch.nn.Linear):
                with torch.no_grad():
                    m.weight.mul_(0.5)
        return f.to(torch.bfloat16).to(DEV)

    plain, fused = ffn(), ffn()
    assert convert_to_fp8(plain) == (3, 3)
    assert convert_to_fp8(fused, fuse_gelu=True) == (3, 3)
    assert isinstance(fused[1], torch.nn.Identity) and fused[2].gelu_input
    assert isinstance(fused[3], torch.nn.GELU) and not fused[4].gelu_input   # the erf form is left alone
    assert not plain[2].gelu_input and isinstance(plain[1], torch.nn.GELU)
    x = torch.randn(2, 300, 1536, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        a, b = plain(x), fused(x)
    torch.cuda.synchronize()
    e = (a.float() - b.float()).abs()
    scale = a.float().abs().max().item()
    record(f"FFN with fused GELU vs unfused: max {e.max().item():.2e} (|out| max {scale:.2e})")
    assert e.max().item() <= 2e-2 * scale
    # an FP8Linear with gelu_input on an fp32 activation takes torch's GELU, then the plain quantisation
    lin = FP8Linear(torch.nn.Linear(1536, 1536).to(torch.bfloat16).to(DEV), gelu_input=True)
    xf = torch.randn(64, 1536, generator=g).to(DEV)
    want = FP8Linear(torch.nn.Linear(1536, 1536).to(torch.bfloat16).to(DEV))
    want.w8, want.w_scale_t, want.bias = lin.w8, lin.w_scale_t, lin.bias
    assert torch.equal(lin(xf), want(torch.nn.functional.gelu(xf, approximate="tanh")))
