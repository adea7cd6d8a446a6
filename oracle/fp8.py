"""CPU restatement of the rowwise FP8 quantisation of the FP8 linear layers (test infrastructure only):
lingbot/layers/linear.py:15-26 -- per row scale = max(amax / 448, 1e-12) in fp32, values x / scale in fp32 cast to
e4m3 (round to nearest even; |x / scale| <= 448 up to the rounding of the division, which the cast takes to 448).
Non-finite rows follow torch: a NaN makes the row's scale and every value NaN; an infinity makes the scale inf,
the row's finite values +-0 and the infinity NaN."""
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


def gelu_tanh_bf16(x):
    """nn.GELU(approximate='tanh') of bf16 x, exact then rounded to bf16 (the module's output on bf16 input,
    lingbot/models/lingbot_world/transformer.py:313-315): 0.5 x (1 + tanh(sqrt(2 / pi) (x + 0.044715 x^3))) in
    fp64, so the result is the correctly rounded bf16 value (torch evaluates it in fp32 and agrees to within a bf16
    ulp). Non-finite inputs: +inf -> inf, -inf -> NaN (0.5 x (1 + tanh) = -inf * 0), NaN -> NaN."""
    xd = x.double()
    inner = (2.0 / torch.pi) ** 0.5 * (xd + 0.044715 * xd * xd * xd)
    g = 0.5 * xd * (1.0 + torch.tanh(inner))
    # fp64 -> bf16 rounded once: through fp32 a value can land exactly on a bf16 tie that the fp64 value is not
    # on; such fp32 values are moved one fp32 ulp toward the fp64 value first, so the tie breaks the right way
    f = g.float()
    tie = ((f.view(torch.int32) & 0xFFFF) == 0x8000) & (f.double() != g)
    toward = torch.where(g > f.double(), torch.tensor(float("inf")), torch.tensor(float("-inf")))
    f = torch.where(tie, torch.nextafter(f, toward), f)
    return f.to(torch.bfloat16)


def quant_mx(x):
    """MXFP8 (lingbot/layers/linear.py:42-50) with the scale exponent taken exactly: x [rows, cols] bf16 / fp32,
    cols a multiple of 32 -> (e4m3 bits uint8 [rows, cols], E8M0 bytes uint8 [rows, cols / 32]). Per 32 values:
    q = fp32(max(amax, 2^-126) / 448), e = ceil(log2(q)) from q's frexp (f = 0.5 exactly: a power of two),
    floored at -127; values e4m3(x / 2^e). The reference evaluates ceil(log2(q)) in fp32, which agrees except when
    q is within an ulp above a power of two and its log2 rounds down onto the integer."""
    m, k = x.shape
    xb = x.float().view(m, k // 32, 32)
    amax = xb.abs().amax(-1).clamp(min=2.0 ** -126)   # NaN if the group holds one (torch's amax propagates it)
    q = amax / torch.tensor(FMAX, dtype=torch.float32)
    f, ex = torch.frexp(q)
    e = torch.where(f == 0.5, ex - 1, ex).clamp(min=-127)
    # a group holding a NaN or an infinity: the reference's scale is NaN / inf (its E8M0 byte 255) and x / scale
    # is NaN, or +-0 for the finite values of an infinite group
    finite = torch.isfinite(amax)
    scale = torch.where(finite, torch.ldexp(torch.ones_like(q), e), amax)
    y = (xb / scale[..., None]).clamp(-FMAX, FMAX)
    e8 = torch.where(finite, e + 127, torch.full_like(e, 255))
    return y.to(torch.float8_e4m3fn).view(torch.uint8).view(m, k), e8.to(torch.uint8)


def dequant_mx(bits, e8):
    m, k = bits.shape
    v = bits.view(torch.float8_e4m3fn).float().view(m, k // 32, 32)
    return (v * torch.ldexp(torch.ones(m, k // 32), e8.long() - 127)[..., None]).view(m, k)
