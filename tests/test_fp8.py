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
