"""CPU restatement of the rowwise FP8 quantisation of the FP8 linear layers (test infrastructure only):
lingbot/layers/linear.py:15-26 -- per row scale = max(amax / 448, 1e-12) in fp32, values x / scale in fp32 cast to
e4m3 (round to nearest even; |x / scale| <= 448 up to the rounding of the division, which the cast takes to 448)."""
import torch

FMAX = 448.0


def quant_rows(x):
    """x [rows, cols] bf16 or fp32 -> (e4m3 bits uint8 [rows, cols], scale fp32 [rows, 1])."""
    xf = x.float()
    scale = (xf.abs().amax(dim=1, keepdim=True) / FMAX).clamp(min=1e-12)
    y = (xf / scale).clamp(-FMAX, FMAX)
    return y.to(torch.float8_e4m3fn).view(torch.uint8), scale


def dequant_rows(bits, scale):
    return bits.view(torch.float8_e4m3fn).float() * scale
