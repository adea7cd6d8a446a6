"""FP8 linear layers (mirrors lingbot/layers/linear.py): rowwise -- weights in e4m3 with one fp32 scale per
output row, converted once at load; activations quantised per token on every call -- or MXFP8, one power-of-two
scale per 32 values along K for both; the GEMM accumulates in fp32 and writes bf16.

On MI355X the per-row quantisation of weights and activations is a HIP kernel (lbw_quant_rows_fp8, bit for bit the
reference's formula) and the GEMM is hipBLASLt's rowwise-scaled FP8 GEMM, reached through torch._scaled_mm with the
bias in its epilogue -- a plain library GEMM, which the dense FP8 MFMA path of the library already serves well.
"""
import torch

from .. import kernels

__all__ = ["FP8Linear", "MXFP8Linear", "convert_to_fp8"]


class FP8Linear(torch.nn.Module):
    """Rowwise FP8 replacement of an nn.Linear (lingbot/layers/linear.py:10-29)."""
    FMAX = torch.finfo(torch.float8_e4m3fn).max

    def __init__(self, lin):
        super().__init__()
        w = lin.weight.detach()
        if w.dtype not in (torch.bfloat16, torch.float32):
            w = w.float()
        w8, w_scale = kernels.quant_rows_fp8(w.contiguous())          # [N, K], [N, 1]
        self.register_buffer("w8", w8)
        self.register_buffer("w_scale_t", w_scale.t().contiguous())   # [1, N]
        self.bias = lin.bias
        self.in_features, self.out_features = lin.in_features, lin.out_features

    def forward(self, x):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.dtype not in (torch.bfloat16, torch.float32):
            x2 = x2.float()
        x8, x_scale = kernels.quant_rows_fp8(x2.contiguous())
        y = torch._scaled_mm(x8, self.w8.t(), scale_a=x_scale, scale_b=self.w_scale_t,
                             bias=None if self.bias is None else self.bias.to(torch.bfloat16),
                             out_dtype=torch.bfloat16)
        return y.reshape(*shape[:-1], y.shape[-1])


MX_ROWS = 128   # hipBLASLt's MX-scaled GEMM takes row counts in multiples of its 128-row tile


def _pad(n, m):
    return (n + m - 1) // m * m


class MXFP8Linear(torch.nn.Module):
    """MXFP8 replacement of an nn.Linear (lingbot/layers/linear.py:53-73): e4m3 with one power-of-two (E8M0)
    scale per 32 values along K for the weights (once) and the activations (every call). The quantisation is
    lbw_quant_mx_fp8; the GEMM is hipBLASLt's MX-scaled FP8 GEMM, whose row counts are padded to 128 (the
    quantiser writes the padding rows, so nothing is copied), the bias added after it as the reference does."""

    def __init__(self, lin):
        super().__init__()
        w = lin.weight.detach()
        if w.dtype not in (torch.bfloat16, torch.float32):
            w = w.float()
        n = w.shape[0]
        w8, ws = kernels.quant_mx_fp8(w.contiguous(), _pad(n, MX_ROWS))
        self.register_buffer("w8", w8)             # [Np, K]
        self.register_buffer("w_scale", ws)        # [Np, K / 32] e8m0
        self.bias = lin.bias
        self.in_features, self.out_features = lin.in_features, lin.out_features

    def forward(self, x):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.dtype not in (torch.bfloat16, torch.float32):
            x2 = x2.float()
        m = x2.shape[0]
        x8, xs = kernels.quant_mx_fp8(x2.contiguous(), _pad(m, MX_ROWS))
        y = torch._scaled_mm(x8, self.w8.t(), scale_a=xs, scale_b=self.w_scale, out_dtype=torch.bfloat16)
        y = y[:m, :self.out_features]
        if self.bias is not None:
            y = y + self.bias.to(torch.bfloat16)
        return y.reshape(*shape[:-1], self.out_features)


def convert_to_fp8(blocks, mx=False):
    """Swap the large nn.Linear layers inside `blocks` for FP8Linear (or MXFP8Linear), by the reference's rule
    (lingbot/layers/linear.py:76-89): both features >= 1024, in_features a multiple of 16 (32 for MX),
    out_features a multiple of 16. Returns (fp8 count, linear count)."""
    n_all, n_fp8 = 0, 0
    for parent in list(blocks.modules()):
        for name, m in list(parent.named_children()):
            if not isinstance(m, torch.nn.Linear):
                continue
            n_all += 1
            if (m.in_features >= 1024 and m.out_features >= 1024
                    and m.in_features % (32 if mx else 16) == 0 and m.out_features % 16 == 0):
                setattr(parent, name, (MXFP8Linear if mx else FP8Linear)(m))
                n_fp8 += 1
    return n_fp8, n_all
