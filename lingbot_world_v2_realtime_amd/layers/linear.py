"""FP8 linear layers (mirrors lingbot/layers/linear.py): rowwise -- weights in e4m3 with one fp32 scale per
output row, converted once at load; activations quantised per token on every call -- or MXFP8, one power-of-two
scale per 32 values along K for both; the GEMM accumulates in fp32 and writes bf16.

On MI355X the per-row quantisation of weights and activations is a HIP kernel (lbw_quant_rows_fp8, bit for bit the
reference's formula) and the GEMM is hipBLASLt's rowwise-scaled FP8 GEMM, reached through torch._scaled_mm with the
bias in its epilogue -- a plain library GEMM, which the dense FP8 MFMA path of the library already serves well.
For the shapes in fp8_gemm_solutions.csv, use_tuned_gemms() makes the GEMM take the hipBLASLt solution measured
fastest for that shape instead of the library's default pick (tune_gemms() writes such a table).
"""
import os

import torch

from .. import kernels

__all__ = ["FP8Linear", "MXFP8Linear", "convert_to_fp8", "fp8_eligible", "use_tuned_gemms", "tune_gemms",
           "GEMM_TABLE"]

# hipBLASLt solutions for the DiT's rowwise FP8 GEMMs at the chunk shape (6032 tokens), as a TunableOp results file:
# a key per (layout, N, M, K, leading dims, rowwise scales, bias type), the solution, its measured time, and the
# torch / HIP / hipBLASLt versions and GPU it holds for. Only the 8960 -> 1536 feed-forward projection is listed:
# its tuned solution runs in 74-76 us against 96-97 us for the default pick; for 1536 -> 1536 and 1536 -> 8960 the
# tuned solutions were no faster in use (27.8 vs 26.6 us, 105.4 vs 105.2 us), so those keep the default.
GEMM_TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fp8_gemm_solutions.csv")


def use_tuned_gemms(path=GEMM_TABLE):
    """Make torch._scaled_mm take the solution `path` records for each GEMM shape in it (torch's TunableOp, read
    only: nothing is measured or written). Other shapes keep hipBLASLt's default; a table recorded with other
    library versions or on another GPU is rejected by TunableOp's validators. Process-wide. Returns whether the
    table was read."""
    import torch.cuda.tunable as tunable
    tunable.enable(True)
    tunable.tuning_enable(False)
    tunable.record_untuned_enable(False)
    return bool(tunable.read_file(path))


def tune_gemms(shapes, path, device="cuda", bias=True):
    """Measure hipBLASLt's solutions for rowwise FP8 GEMMs of the given (M, K, N) shapes (an [M, K] activation times
    the [N, K] weight of an FP8Linear, bf16 out, with a bf16 bias when `bias`) and write the fastest of each into
    the TunableOp results file `path`. Tuning stays on for the process afterwards; read the table back with
    use_tuned_gemms() in the process that runs the model. TunableOp writes the file (by the time the process ends)."""
    import torch.cuda.tunable as tunable
    tunable.enable(True)
    tunable.tuning_enable(True)
    tunable.set_filename(path)
    for m, k, n in shapes:
        x8 = torch.randn(m, k, device=device).to(torch.float8_e4m3fn)
        w8 = torch.randn(n, k, device=device).to(torch.float8_e4m3fn)
        xs = torch.ones(m, 1, device=device)
        ws = torch.ones(1, n, device=device)
        b = torch.zeros(n, device=device, dtype=torch.bfloat16) if bias else None
        torch._scaled_mm(x8, w8.t(), scale_a=xs, scale_b=ws, bias=b, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    return tunable.get_results()


class FP8Linear(torch.nn.Module):
    """Rowwise FP8 replacement of an nn.Linear (lingbot/layers/linear.py:10-29). gelu_input: the module also
    applies the GELU (tanh form) that precedes it in a feed-forward block, fused into the activation quantisation
    (lbw_quant_rows_fp8_gelu) for bf16 activations; convert_to_fp8(..., fuse_gelu=True) sets it."""

    def __init__(self, lin, gelu_input=False):
        super().__init__()
        self.gelu_input = bool(gelu_input)
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
        if self.gelu_input and x2.dtype == torch.bfloat16:
            x8, x_scale = kernels.quant_rows_fp8_gelu(x2.contiguous())
        else:
            if self.gelu_input:   # another input type: the GELU in that type first, as the unfused module runs it
                x2 = torch.nn.functional.gelu(x2, approximate="tanh")
            if x2.dtype not in (torch.bfloat16, torch.float32):
                x2 = x2.float()
            x8, x_scale = kernels.quant_rows_fp8(x2.contiguous())
        y = torch._scaled_mm(x8, self.w8.t(), scale_a=x_scale, scale_b=self.w_scale_t,
                             bias=None if self.bias is None else self.bias.to(torch.bfloat16),
                             out_dtype=torch.bfloat16)
        return y.reshape(*shape[:-1], y.shape[-1])


MX_ROWS = 128   # hipBLASLt's MX-scaled GEMM takes row counts in multiples of its 128-row tile
MX_K = 128      # and K in whole 128-value tiles: four E8M0 scale columns (the reference pads its scales to this too)


def _pad(n, m):
    return (n + m - 1) // m * m


class MXFP8Linear(torch.nn.Module):
    """MXFP8 replacement of an nn.Linear (lingbot/layers/linear.py:53-73): e4m3 with one power-of-two (E8M0)
    scale per 32 values along K for the weights (once) and the activations (every call). The quantisation is
    lbw_quant_mx_fp8; the GEMM is hipBLASLt's MX-scaled FP8 GEMM, whose row counts are padded to 128 (the
    quantiser writes the padding rows, so nothing is copied), the bias added after it as the reference does.
    A K that is not a multiple of 128 (the GEMM's scale tile) is padded with zero columns, weights once and
    activations per call: a zero group quantises to zeros, so the product is unchanged."""

    def __init__(self, lin):
        super().__init__()
        w = lin.weight.detach()
        if w.dtype not in (torch.bfloat16, torch.float32):
            w = w.float()
        n, k = w.shape
        self.k_pad = _pad(k, MX_K) - k
        if self.k_pad:
            w = torch.nn.functional.pad(w, (0, self.k_pad))
        w8, ws = kernels.quant_mx_fp8(w.contiguous(), _pad(n, MX_ROWS))
        self.register_buffer("w8", w8)             # [Np, Kp]
        self.register_buffer("w_scale", ws)        # [Np, Kp / 32] e8m0
        self.bias = lin.bias
        self.in_features, self.out_features = lin.in_features, lin.out_features

    def forward(self, x):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.dtype not in (torch.bfloat16, torch.float32):
            x2 = x2.float()
        if self.k_pad:
            x2 = torch.nn.functional.pad(x2, (0, self.k_pad))
        m = x2.shape[0]
        x8, xs = kernels.quant_mx_fp8(x2.contiguous(), _pad(m, MX_ROWS))
        y = torch._scaled_mm(x8, self.w8.t(), scale_a=xs, scale_b=self.w_scale, out_dtype=torch.bfloat16)
        y = y[:m, :self.out_features]
        if self.bias is not None:
            y = y + self.bias.to(torch.bfloat16)
        return y.reshape(*shape[:-1], self.out_features)


def fp8_eligible(lin, mx=False):
    """The reference's rule for which linears run in FP8 (lingbot/layers/linear.py:76-89): both dimensions at
    least 1024, out_features a multiple of 16 and in_features a multiple of 16 (of 32, the scale group, for MX)."""
    k_mult = 32 if mx else 16
    return min(lin.in_features, lin.out_features) >= 1024 and lin.out_features % 16 == 0 and \
        lin.in_features % k_mult == 0


def convert_to_fp8(blocks, mx=False, fuse_gelu=False):
    """Replace every eligible nn.Linear below `blocks` (fp8_eligible) by FP8Linear, or MXFP8Linear with mx=True,
    in place. Returns (replaced, linears seen). fuse_gelu (rowwise only): inside an nn.Sequential, a tanh-form
    nn.GELU directly followed by a replaced linear -- the DiT's feed-forward block,
    lingbot/models/lingbot_world/transformer.py:313-315 -- becomes nn.Identity and the linear applies the GELU in
    its activation quantisation (FP8Linear gelu_input), one pass over the activation instead of two."""
    make = MXFP8Linear if mx else FP8Linear
    found = [(path, m) for path, m in blocks.named_modules() if path and isinstance(m, torch.nn.Linear)]
    chosen = [(path, m) for path, m in found if fp8_eligible(m, mx)]
    for path, m in chosen:
        owner, _, attr = path.rpartition(".")
        setattr(blocks.get_submodule(owner), attr, make(m))
    if fuse_gelu and not mx:
        for seq in [m for m in blocks.modules() if isinstance(m, torch.nn.Sequential)]:
            kids = list(seq)
            for i in range(len(kids) - 1):
                act, lin = kids[i], kids[i + 1]
                if isinstance(act, torch.nn.GELU) and act.approximate == "tanh" and isinstance(lin, FP8Linear):
                    lin.gelu_input = True
                    seq[i] = torch.nn.Identity()
    return len(chosen), len(found)
