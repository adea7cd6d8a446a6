"""Pure-torch CPU emulation of the quantized attention scheme (the oracle; test infrastructure only).

This restates, on the CPU, the arithmetic the HIP kernels implement, so that the int8 Q/K tensors, every
scale, the K smoothing mean, the fp8 V bytes and the int32 QK^T logits can be compared bit for bit, and the
attention output within tolerance. It follows the reference's own pure-torch restatement of SageAttention's
quantisers and its documentation of the fused kernel:

- Q: int8 per 32-row group of 128-row tiles, scale = amax / 127, amax floored at 1e-7, values
  x * (127 / amax) in fp32, round half to even, saturate; rows past Lq count as zero
  (experiments/modules/sage_kvq.py:57-66, :104; rounding statement :14-19).
- K: subtract the per-(head, channel) mean over the chunk, rounded to the input's dtype (bf16, or fp16) as
  `k.mean(dim=1)` on such a tensor is (lingbot/layers/sage_preq.py:115; sage_kvq.py:85, :96), then int8 per
  64-token block as above;
  tokens past the chunk count as zero after the subtraction (sage_kvq.py:61-63).
- V: fp8 e4m3 with per-channel scales (sage_kvq.py:69-75; sage_preq.py:47-78), here one per (head, channel) for
  each 32-key half of a 64-key block. The reference maps the channel's amax to 2.25 because its PV accumulates
  in fp16 (sage_kvq.py:30-31); the MFMA here accumulates in fp32, so the scale is the power of two 2^e that takes
  the group's amax into (224, 448], the top binade of e4m3: V / 2^e is exact, e4m3's relative precision is the
  same in every binade, and a power-of-two scale rides on the fp8 MFMA's E8M0 block-scale operand (per A row and
  32-key block) instead of a multiply of the accumulator. A group's scale needs only its own block, so a chunk's
  V is quantised in one pass over it. A second plane carries the residual y - hi of y = V / 2^e as bf6 (OCP
  e3m2) codes, which the attention multiplies by bf6(P / 16) on the 6-bit MFMA (at twice the fp8 rate).
- Logits: S = q8 . k8 in int32 (experiments/bench_attn/h2_tiles/README.md:45), dequantised with
  q_scale * k_scale * sm_scale * log2(e) into the exp2 domain; P = exp2(s - m + 8.807) <= 448 cast to e4m3
  (experiments/bench_attn/phi_calib.md:11-16); O = sum P V / sum P, with the V scale
  (h2_tiles/README.md:13-20; experiments/bench_attn/splitkv/README.md:62-63). The reference max m of a row
  moves only when a block's max passes it by more than RESCALE_SLACK, so the rescale of the accumulated O is
  rare; each block's contribution is accumulated in true V units (its power-of-two group scales applied by the
  MFMA), so nothing is rescaled between blocks or chunks.
- Memory chunks keep their own mean and V scale; the bias q . mean_c of chunk c is added to its logits
  (a constant per (query, chunk), so it drops out when there is only one chunk).

Order of the K mean (fixed so it is reproducible bit for bit): token t of a chunk sits in 64-token block
b = t // 64 at row r = t % 64 = 4 q + j (q in 0..15, j in 0..3); blocks form super-blocks of 4 (u = b // 4).
In fp32, every sum starting from +0 and running left to right:
  s[b, q]  = x[4q] + x[4q + 1] + x[4q + 2] + x[4q + 3]
  H[b, i]  = s[b, 8i] + s[b, 8i + 1] + ... + s[b, 8i + 7]   (the two 32-token halves, i = 0, 1)
  B[b]     = H[b, 0] + H[b, 1]
  U[u]     = B[4u] + B[4u + 1] + B[4u + 2] + B[4u + 3]     (the blocks that exist)
  total    = U[0] + U[1] + ... + U[nsup - 1]
  mean     = total / n (fp32, correctly rounded), km = mean rounded to nearest even in the input's dtype
             (bf16, or fp16 for fp16 K).
Padding tokens past n add +0.

fp8 V layout per 64-key block: [channel][64 positions]; position p holds key
  key(p) = 32 * ((p & 31) >> 4) + 8 * ((p >> 2) & 3) + 4 * (p >> 5) + (p & 3),
the order in which an MFMA 32x32 int32 output tile of S^T (two tiles per 64 keys) leaves the keys in the
lanes that then feed P^T to the fp8 PV MFMA, so P needs no reordering between the two products.
"""
import numpy as np
import torch

Q_GROUP = 32            # query rows per Q scale
Q_TILE = 256            # Lq is padded to whole tiles of this many rows (the attention tile)
K_BLOCK = 64            # keys per K scale and per V block
SUPER_BLOCK = 4         # K blocks per partial sum of the mean
HEAD_DIM = 128
V_MAX = 448.0           # e4m3 max; the V scale maps amax to it
AMAX_FLOOR = 1e-7
P_OFFSET = 8.807        # log2(448): P = exp2(s - m + P_OFFSET) <= 448
V_TERMS = 2             # V terms: hi = e4m3(y), and the residual plane lo = bf6(y - hi)
P_LO_SCALE = 16.0       # the residual product takes P as bf6(P / 16); the MFMA's B scale 2^4 restores the factor
V_LO_ROW = 48           # bytes of one channel's 64 bf6 residual codes in a block
RESCALE_SLACK = 2.0     # tau: a row's reference max moves only when a block max exceeds it by more than tau
LOG2E = 1.4426950408889634


def pad_to(n, m):
    return (n + m - 1) // m * m


def key_of_position(p):
    """Key index (0..63) held at position p of a 64-key fp8 V block."""
    p = np.asarray(p)
    return 32 * ((p & 31) >> 4) + 8 * ((p >> 2) & 3) + 4 * (p >> 5) + (p & 3)


def position_of_key(k):
    """Inverse of key_of_position."""
    k = np.asarray(k)
    return 32 * ((k >> 2) & 1) + 16 * ((k >> 5) & 1) + 4 * ((k >> 3) & 3) + (k & 3)


V_KEY_OF_POS = key_of_position(np.arange(64))
V_POS_OF_KEY = position_of_key(np.arange(64))


def bf16_round(x):
    """fp32 -> nearest bf16 (ties to even), returned as fp32."""
    return x.to(torch.bfloat16).to(torch.float32)


def e4m3_encode(x):
    """fp32 tensor (|x| <= 448) -> e4m3fn bits (uint8), round to nearest even."""
    return x.clamp(-V_MAX, V_MAX).to(torch.float8_e4m3fn).view(torch.uint8)


def e4m3_encode_nonfinite(x):
    """e4m3_encode for values within e4m3's range, a NaN or an infinity as the NaN code 0x7F (with its sign bit)."""
    bad = ~torch.isfinite(x)
    bits = e4m3_encode(torch.where(bad, torch.zeros_like(x), x))
    return torch.where(bad, (torch.signbit(x).to(torch.uint8) << 7) | 0x7F, bits)


def e4m3_decode(bits):
    """e4m3fn bits (uint8) -> fp32."""
    return bits.view(torch.float8_e4m3fn).to(torch.float32)


def bf6_encode(x):
    """fp32 tensor -> bf6 codes (OCP e3m2: sign in bit 5, exponent bits 4:2 with bias 3, mantissa bits 1:0, no inf
    or NaN codes) as uint8 0..63, rounded to nearest even the way gfx950's v_cvt_scalef32_2xpk16_bf6_f32 converts:
    magnitudes above 28 and infinities saturate to 28, a NaN becomes 28 with the NaN's sign bit, and a value that
    rounds to zero keeps its sign. The step is 2^(e - 2) in the binade [2^e, 2^(e + 1)), e = -2 .. 4, and 2^-4
    below 0.25 (the subnormals)."""
    a = x.abs().to(torch.float32)
    a = torch.where(torch.isnan(a), torch.full_like(a, 32.0), a.clamp_max(32.0))   # 32 saturates below
    _, ex = torch.frexp(a)                                          # a in [2^(ex - 1), 2^ex)
    eb = torch.where(a < 0.25, torch.full_like(ex, -2), ex - 1).clamp_max(4)
    q = torch.round(torch.ldexp(a, 2 - eb))                         # 4..8 in a normal binade, 0..4 below
    mag = (4 * (eb + 2) + q.to(torch.int32)).clamp_max(31)          # q = 8 carries into the next binade
    return (mag | (torch.signbit(x).to(torch.int32) << 5)).to(torch.uint8)


def bf6_round(x):
    """bf6_decode(bf6_encode(x)) for finite fp32 x, as values, computed faster: in bf6's normal range (0.25 and up)
    its rounding is that of e5m2 (the same 2 mantissa bits, to nearest even), saturating at 28; below 0.25 it is
    the multiple of 2^-4 nearest x (ties to even), which keeps the sign of x."""
    e5 = x.clamp(-28.0, 28.0).to(torch.float8_e5m2).to(torch.float32).clamp(-28.0, 28.0)
    sub = torch.round(x * 16.0) / 16.0
    return torch.where(x.abs() < 0.25, sub, e5)


def bf6_decode(bits):
    """bf6 (e3m2) codes (uint8 0..63) -> fp32."""
    b = bits.to(torch.int32)
    e, m = (b >> 2) & 7, (b & 3).to(torch.float32)
    mag = torch.where(e > 0, (4.0 + m) * torch.ldexp(torch.ones_like(m), e - 5), m / 16.0)
    return torch.where((b >> 5) & 1 == 1, -mag, mag)


BF6_POS_OF_CODE = np.array([16 * g + c + (c & 16) for g in range(2) for c in range(32)])   # [group g][code c]


def pack_bf6_rows(codes):
    """bf6 codes [..., C, 64 positions] (C channels) -> packed rows uint8 [..., C, 48]. Group g holds the positions
    of V scale group g (16 g .. 16 g + 15 and 32 + 16 g .. 47 + 16 g, the keys 32 g .. 32 g + 31): its code c is
    position 16 g + c + (c & 16), because a lane of the 6-bit MFMA operand holds one whole K-block (lane half g:
    K-block g), where an fp8 lane holds 16 values of each. A group's 32 codes are 24 bytes, code c at bits
    6 c .. 6 c + 5 little endian; a row is group 0's bytes 0-15, group 1's bytes 0-15, then the two 8-byte tails
    (bytes 16-23 of each group): group 0's first in channels whose bit 4 is clear, group 1's first where it is set.
    A lane reads its group's 24 bytes as one 16-byte and one 8-byte LDS load; at the 48-byte row stride the 16-byte
    loads of 16 consecutive channels cover the 64 banks once, and with the tails swapped so do the 8-byte loads
    of 32."""
    c = codes.to(torch.int64)[..., torch.from_numpy(BF6_POS_OF_CODE)].reshape(*codes.shape[:-1], 2, 8, 4)
    w = c[..., 0] | (c[..., 1] << 6) | (c[..., 2] << 12) | (c[..., 3] << 18)      # 4 codes = 3 bytes
    b = torch.stack([w & 255, (w >> 8) & 255, (w >> 16) & 255], dim=-1).reshape(*codes.shape[:-1], 2, 24)
    swap = (((torch.arange(codes.shape[-2]) >> 4) & 1) == 1)[:, None]
    t0 = torch.where(swap, b[..., 1, 16:], b[..., 0, 16:])
    t1 = torch.where(swap, b[..., 0, 16:], b[..., 1, 16:])
    return torch.cat([b[..., 0, :16], b[..., 1, :16], t0, t1], dim=-1).to(torch.uint8)


def unpack_bf6_rows(rows):
    """Inverse of pack_bf6_rows: uint8 [..., C, 48] -> codes [..., C, 64]."""
    r = rows.to(torch.int64)
    swap = (((torch.arange(rows.shape[-2]) >> 4) & 1) == 1)[:, None]
    t0 = torch.where(swap, r[..., 40:48], r[..., 32:40])
    t1 = torch.where(swap, r[..., 32:40], r[..., 40:48])
    halves = torch.stack([torch.cat([r[..., 0:16], t0], -1), torch.cat([r[..., 16:32], t1], -1)], -2)
    b = halves.reshape(*rows.shape[:-1], 2, 8, 3)
    w = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16)
    c = torch.stack([(w >> (6 * i)) & 63 for i in range(4)], dim=-1).reshape(*rows.shape[:-1], 64)
    out = torch.empty_like(c)
    out[..., torch.from_numpy(BF6_POS_OF_CODE)] = c
    return out.to(torch.uint8)


def _as_lhd(x):
    """Accept [L, H, D] or [1, L, H, D]; return [L, H, D]."""
    if x.dim() == 4:
        assert x.shape[0] == 1, "the oracle handles batch 1; loop over the batch outside"
        x = x[0]
    return x


def _quant_int8_blocks(xf, blk):
    """xf: fp32 [H, nblk, blk, D] (padding already zero) -> int8 same shape, scale fp32 [H, nblk]."""
    amax = xf.abs().amax(dim=(2, 3)).clamp_min(AMAX_FLOOR)
    recip = torch.full_like(amax, 127.0) / amax                  # fp32, correctly rounded
    q = (xf * recip[:, :, None, None]).round().clamp(-128, 127).to(torch.int8)
    scale = amax / torch.full_like(amax, 127.0)
    return q, scale


def quant_q(q):
    """q bf16 [Lq, H, D] -> (q8 int8 [H, Lp, D], q_scale fp32 [H, Lp / 32]); Lp = Lq rounded up to 256 (Q_TILE)."""
    q = _as_lhd(q)
    lq, h, d = q.shape
    lp = pad_to(lq, Q_TILE)
    xf = torch.zeros(h, lp, d, dtype=torch.float32)
    xf[:, :lq] = q.float().permute(1, 0, 2)
    q8, qs = _quant_int8_blocks(xf.view(h, lp // Q_GROUP, Q_GROUP, d), Q_GROUP)
    return q8.view(h, lp, d), qs


def chunk_mean(k, rounded=True):
    """Per-(head, channel) mean of k bf16 / fp16 [L, H, D] in the fixed order above -> fp32 [H, D] holding values
    of k's dtype (the mean is rounded to it, as `k.mean(dim=1)` on a bf16 or fp16 tensor is); rounded=False returns
    the fp32 mean before that rounding."""
    k = _as_lhd(k)
    n, h, d = k.shape
    nb = pad_to(n, K_BLOCK) // K_BLOCK
    x = torch.zeros(nb * K_BLOCK, h, d, dtype=torch.float32)
    x[:n] = k.float()
    x = x.view(nb, 16, 4, h, d)                  # [b, q, j, h, d]: token = 64 b + 4 q + j
    s = torch.zeros(nb, 16, h, d, dtype=torch.float32)
    for j in range(4):
        s = s + x[:, :, j]
    half = torch.zeros(nb, 2, h, d, dtype=torch.float32)
    for q in range(8):
        half = half + s[:, q::8]
    blk = half[:, 0] + half[:, 1]
    tot = torch.zeros(h, d, dtype=torch.float32)
    for u in range(0, nb, SUPER_BLOCK):
        sup = torch.zeros(h, d, dtype=torch.float32)
        for b in range(u, min(nb, u + SUPER_BLOCK)):
            sup = sup + blk[b]
        tot = tot + sup
    mean = tot / torch.tensor(float(n), dtype=torch.float32)
    if not rounded:
        return mean
    return mean.to(k.dtype).to(torch.float32) if k.dtype in (torch.bfloat16, torch.float16) else bf16_round(mean)


def quant_k(k, km):
    """k bf16 [L, H, D], km fp32 [H, D] -> (k8 int8 [H, Lp64, D], k_scale fp32 [H, nb])."""
    k = _as_lhd(k)
    n, h, d = k.shape
    lp = pad_to(n, K_BLOCK)
    xf = torch.zeros(h, lp, d, dtype=torch.float32)
    xf[:, :n] = k.float().permute(1, 0, 2) - km[:, None, :]
    k8, ks = _quant_int8_blocks(xf.view(h, lp // K_BLOCK, K_BLOCK, d), K_BLOCK)
    return k8.view(h, lp, d), ks


V_GROUP_OF_KEY = np.arange(K_BLOCK) >> 5   # key group of in-block key k: its 32-key half (see quant_v)


def v_group_exponents(v):
    """v [L, H, D] -> e int64 [H, nb, 2, D]: per 64-key block, key group g and channel, the exponent of the power of
    two 2^e with amax / 2^e in (224, 448], amax over the group's 32 keys (padding tokens count as zero; floored at
    1e-7). With amax = f * 2^x, f in [0.5, 1): e = x - 9 when f <= 0.875 (448 = 0.875 * 2^9), else x - 8 -- integer
    arithmetic on the exponent, no rounding. A NaN does not enter the amax (the kernel's max skips it); an infinite
    amax takes the kernel's bit rule for the exponent field 255, x = 129: e = 120."""
    v = _as_lhd(v)
    n, h, d = v.shape
    lp = pad_to(n, K_BLOCK)
    x = torch.zeros(h, lp, d, dtype=torch.float32)
    x[:, :n] = v.float().abs().nan_to_num(nan=0.0, posinf=float("inf")).permute(1, 0, 2)
    x = x.view(h, lp // K_BLOCK, K_BLOCK, d)
    grp = torch.from_numpy(V_GROUP_OF_KEY)
    amax = torch.stack([x[:, :, grp == g].amax(dim=2) for g in (0, 1)], dim=2).clamp_min(AMAX_FLOOR)
    f, ex = torch.frexp(amax)
    e = torch.where(f <= 0.875, ex - 9, ex - 8).long()
    return torch.where(amax.isinf(), torch.full_like(e, 120), e)


def v_scale_table(e):
    """e [H, nb, 2, D] -> the E8M0 scale bytes uint8 [H, nb, 256] of each block in the attention's lane order:
    byte (32 g + lq) * 4 + mt = 127 + e[g][32 mt + lq], the scale of channel 32 mt + lq for the keys of group g."""
    h, nb = e.shape[:2]
    t = (e + 127).view(h, nb, 2, 4, 32)               # [h, b, g, mt, lq]: channel = 32 mt + lq
    return t.permute(0, 1, 2, 4, 3).reshape(h, nb, 256).to(torch.uint8)


def v_exponents_of_table(table):
    """Inverse of v_scale_table: uint8 [H, nb, 256] -> e int64 [H, nb, 2, D]."""
    h, nb = table.shape[:2]
    return table.long().view(h, nb, 2, 32, 4).permute(0, 1, 2, 4, 3).reshape(h, nb, 2, HEAD_DIM) - 127


def quant_v(v):
    """v bf16 / fp16 [L, H, D] -> (v8 uint8 e4m3 bits [H, nb, D, 64] in the permuted key order, v8lo the residual
    plane uint8 [H, nb, D, 48] of bf6 codes over the same positions (pack_bf6_rows), the E8M0 scale table uint8
    [H, nb, 256] of v_scale_table).

    Scales are powers of two, one per (64-key block, key group, channel): group g of a block holds its keys
    32 g .. 32 g + 31, the 32-deep K-block g of the 64-deep PV MFMA (bytes 16 g .. 16 g + 15 of every lane's fp8
    operand, which the permuted layout fills with those keys; all 32 codes of lane half g's 6-bit operand, which
    pack_bf6_rows fills with them), whose E8M0 block scale of the A operand applies per row and K-block -- so the
    MFMA applies the scale itself. Two terms:
    y = v / 2^e (exact, |y| <= 448); hi = e4m3(y); lo = bf6(y - hi), so v ~ (hi + lo) * 2^e. y - hi is exact in
    fp32 (hi is y rounded to 3 mantissa bits) and |y - hi| <= 16 (half an e4m3 step below 448) lies inside bf6's
    range, so lo needs no scale of its own. A NaN or an infinity in V gives hi a NaN code and lo the code of 28
    (bf6 has no NaN; the sign is the NaN residual's)."""
    v = _as_lhd(v)
    n, h, d = v.shape
    lp = pad_to(n, K_BLOCK)
    e = v_group_exponents(v)
    per_key = e[:, :, torch.from_numpy(V_GROUP_OF_KEY)]                  # [h, nb, 64 keys, d]
    recip = torch.ldexp(torch.ones(per_key.shape), -per_key).view(h, lp, d)
    y = torch.zeros(h, lp, d, dtype=torch.float32)
    y[:, :n] = v.float().permute(1, 0, 2)
    y = y * recip                                   # |y| <= 448 for finite V: no clamp, a NaN or inf stays one
    hi = e4m3_encode_nonfinite(y)
    lo = bf6_encode(y - e4m3_decode(hi))
    planes = []
    for bits in (hi, lo):
        bits = bits.view(h, lp // K_BLOCK, K_BLOCK, d)[:, :, torch.from_numpy(V_KEY_OF_POS)]   # [h, b, pos, d]
        planes.append(bits.permute(0, 1, 3, 2).contiguous())
    return planes[0], pack_bf6_rows(planes[1]), v_scale_table(e)


def requant(k, v):
    """The save-to-memory re-quant of one chunk: bf16 K, V [L, H, D] -> dict of the quantised chunk."""
    k = _as_lhd(k)
    km = chunk_mean(k)
    k8, ks = quant_k(k, km)
    v8, v8lo, vs = quant_v(v)
    return {"k8": k8, "k_scale": ks, "km": km, "v8": v8, "v8lo": v8lo, "v_scale": vs, "n": k.shape[0]}


def span(chunk):
    """(first, n, first block, blocks) of the keys a quantised chunk is read over: keys [first, first + n) of its
    slot ("first" defaults to 0; "n" is the count read), in the slot's own 64-key blocks, so the first block may
    start before `first` and the last may end past first + n (those keys are masked)."""
    first, n = chunk.get("first", 0), chunk["n"]
    b0 = first // K_BLOCK
    return first, n, b0, pad_to(first + n, K_BLOCK) // K_BLOCK - b0


def dequant_v_planes(chunk):
    """The V planes of a quantised chunk in true units, fp32 [H, first + n, D] each in key order (slot keys
    0 .. first + n - 1): (hi * 2^e, lo * 2^e) with each key's group scale; lo is None for a chunk whose "v8lo" is
    None (quantised without the residual plane)."""
    h, nb, d, _ = chunk["v8"].shape
    end = chunk.get("first", 0) + chunk["n"]
    e = v_exponents_of_table(chunk["v_scale"])[:, :, torch.from_numpy(V_GROUP_OF_KEY)]   # [h, nb, key, d]
    scale = torch.ldexp(torch.ones(e.shape), e)
    pos = torch.from_numpy(V_POS_OF_KEY)
    out = []
    for vals in (e4m3_decode(chunk["v8"]),
                 bf6_decode(unpack_bf6_rows(chunk["v8lo"])) if chunk.get("v8lo") is not None else None):
        if vals is not None:   # [h, nb, d, position] -> [h, keys, d]
            vals = (vals[:, :, :, pos].permute(0, 1, 3, 2) * scale).reshape(h, nb * K_BLOCK, d)[:, :end]
        out.append(vals)
    return out[0], out[1]


def dequant_v(chunk, terms=None):
    """V of a quantised chunk back to fp32 [H, first + n, D] in key order (slot keys 0 .. first + n - 1), in true
    units: (hi + lo) * 2^e with each key's group scale (or hi alone with terms=1, the default for a chunk whose
    "v8lo" is None)."""
    hi, lo = dequant_v_planes(chunk)
    if terms is None:
        terms = V_TERMS if lo is not None else 1
    return hi + lo if terms == 2 else hi


def qk_logits(q8, k8):
    """int32 S = q8 . k8^T: [H, Lq, D] x [H, Lk, D] -> [H, Lq, Lk]. fp32 GEMM of int8 values is exact at
    d = 128 (|S| <= 2^21 < 2^24)."""
    s = torch.matmul(q8.float(), k8.float().transpose(1, 2))
    return s.to(torch.int32)


def q_bias(q, km):
    """q . km in fp32 for every query and head: q bf16 [Lq, H, D], km fp32 [H, D] -> [H, Lq]."""
    q = _as_lhd(q)
    return torch.einsum("lhd,hd->hl", q.float(), km)


def _sl2(sm_scale, d):
    """sm_scale * log2(e) as the fp32 product the kernels use."""
    sm = torch.tensor(d ** -0.5 if sm_scale is None else sm_scale, dtype=torch.float32)
    return sm * torch.tensor(LOG2E, dtype=torch.float32)


XCDS = 8


def attn_schedule(n_tiles, nb, gx):
    """Key-block pieces of every Q_TILE-query tile under the kernel's schedule: tiles (head-major) split into 8
    contiguous per-XCD ranges; within a range whole tiles go round-robin to its `gx` workgroups while each
    gets one, and the rest's (tile, block) units are cut into `gx` equal contiguous pieces.
    Returns {tile: [(j0, j1), ...]} with pieces in increasing j0 (the merge order)."""
    pieces = {t: [] for t in range(n_tiles)}
    for x in range(XCDS):
        t_lo, t_hi = x * n_tiles // XCDS, (x + 1) * n_tiles // XCDS
        ts = t_lo + (t_hi - t_lo) // gx * gx
        units = (t_hi - ts) * nb
        for t in range(t_lo, ts):
            pieces[t].append((0, nb))
        for i in range(gx):
            u, u1 = i * units // gx, (i + 1) * units // gx
            while u < u1:
                t, j0 = ts + u // nb, u % nb
                j1 = min(nb, j0 + (u1 - u))
                pieces[t].append((j0, j1))
                u += j1 - j0
    return pieces


def _attend_blocks(qf, qsr, chunks, vdec, beta_of, hh, j0, j1, sl2, tau, stats=None, p_round=True):
    """Online softmax over tile-relative key blocks [j0, j1) (numbered across the chunks in order) for the
    query rows `qf` (q8 as fp32) -> (o in true V units, m, l). The reference max m of a row moves only when a
    block's max exceeds it by more than `tau`. The row sum l adds up the P that the hi plane's PV product
    multiplies: the e4m3 P (so O / l normalises exactly the weights applied to hi), or with p_round=False the
    unrounded fp32 P. The residual plane's product takes P as bf6(P / 16) * 16, whose rounding (2^-3 relative)
    acts on a term at most 2^-4 of V. The reference's Sage kernel sums the unrounded P instead (a deviation of
    ~2^-5 / sqrt(keys) relative in l)."""
    rows, d = qf.shape[0], qf.shape[1]
    m_run = torch.full((rows,), float("-inf"))
    l_run = torch.zeros(rows)
    o = torch.zeros(rows, d)
    j = 0
    for ci, c in enumerate(chunks):
        first, n, b0, nbc = span(c)
        if j + nbc <= j0 or j >= j1:
            j += nbc
            continue
        beta = beta_of(ci)
        for b in range(max(0, j0 - j), min(nbc, j1 - j)):
            sb = b0 + b   # the slot's block
            k0, k1 = max(first, sb * K_BLOCK), min(first + n, sb * K_BLOCK + K_BLOCK)
            s_int = torch.matmul(qf, c["k8"][hh, k0:k1].float().t())
            cb = (qsr * sl2) * c["k_scale"][hh, sb]
            m_blk = s_int.amax(dim=1) * cb + beta
            m_new = torch.where(m_blk > m_run + tau, m_blk, m_run)
            if stats is not None:
                stats.append(float((m_new != m_run).float().mean()))
            alpha = torch.exp2(m_run - m_new)
            m_run = m_new
            o = o * alpha[:, None]
            l_run = l_run * alpha
            kc = (beta - m_new + (P_OFFSET - tau)).double()
            x = (s_int.double() * cb.double()[:, None] + kc[:, None]).float()
            p = torch.exp2(x)
            pr = e4m3_decode(e4m3_encode(p)) if p_round else p
            l_run = l_run + pr.sum(dim=1)
            # V in true units: its group scales are powers of two, exact, the factors the MFMA's block scale applies
            hi, lo = vdec[ci]
            o = o + torch.matmul(pr, hi[hh, k0:k1])
            if lo is not None:
                pl = bf6_round(p / P_LO_SCALE) * P_LO_SCALE if p_round else p
                o = o + torch.matmul(pl, lo[hh, k0:k1])
        j += nbc
    return o, m_run, l_run


def attention(q, chunks, sm_scale=None, q_block=1024, schedule_gx=None, tau=None, stats=None, p_round=True):
    """Emulated quantized attention of q bf16 [Lq, H, D] over quantised chunks (dicts from `requant`; a chunk is
    read over keys [first, first + n) of its slot, see `span`), in the kernel's own order: chunks in sequence, the
    slot's 64-key blocks in sequence (keys outside the read range masked), a reference row max m, and per block
      b = max_j S_ij * cb + beta,  m_new = b if b > m + tau else m,  alpha = exp2(m - m_new),
      o = alpha * o,  l = alpha * l,  P_ij = exp2(S_ij * cb + beta - m_new + 8.807 - tau)  (<= 448),
      l += sum e4m3(P),  o += e4m3(P) . (hi * 2^e) + bf6(P / 16) * 16 . (lo * 2^e)  (V in true units, its
      group scales applied),
    with cb = q_scale * k_scale * sm_scale * log2(e) and beta = q . mean_k of the chunk (several chunks only);
    finally out = o / l. Each block's contribution is in true V units, so a chunk switch needs no rescale.
    With `schedule_gx` (the kernel's workgroups per XCD), tiles the kernel splits between workgroups are
    computed piece by piece from a fresh state and merged by `merge_partials`.
    p_round=False skips the rounding of P (a checking mode: the result is then exact softmax attention of
    the dequantised logits and V, whatever the block order, running max or split).
    Returns fp32 [Lq, H, D].
    """
    q = _as_lhd(q)
    lq, h, d = q.shape
    tau = RESCALE_SLACK if tau is None else tau
    sl2 = _sl2(sm_scale, d)
    q8, qs = quant_q(q)
    multi = len(chunks) > 1
    vdec = [dequant_v_planes(c) for c in chunks]
    bias = [q_bias(q, c["km"]) * sl2 if multi else None for c in chunks]
    nb = sum(span(c)[3] for c in chunks)
    q_tiles = pad_to(lq, Q_TILE) // Q_TILE
    sched = attn_schedule(q_tiles * h, nb, schedule_gx) if schedule_gx else None
    out = torch.empty(lq, h, d, dtype=torch.float32)
    qsr_all = qs.repeat_interleave(Q_GROUP, dim=1)
    for hh in range(h):
        # row ranges that run as one piece over all blocks, and the split tiles
        split = set()
        if sched is not None:
            split = {t for t in range(q_tiles) if sched[hh * q_tiles + t] != [(0, nb)]}
        ranges, a = [], 0
        while a < lq:
            t = a // Q_TILE
            if t in split:
                ranges.append((a, min(lq, a + Q_TILE), t))
                a += Q_TILE
            else:
                e = min(lq, a + max(Q_TILE, q_block // Q_TILE * Q_TILE))
                for tt in range(t, (e + Q_TILE - 1) // Q_TILE):
                    if tt in split:
                        e = tt * Q_TILE
                        break
                ranges.append((a, e, None))
                a = e
        for a, e, t in ranges:
            qf = q8[hh, a:e].float()
            qsr = qsr_all[hh, a:e]
            beta_of = (lambda ci: bias[ci][hh, a:e]) if multi else (lambda ci: torch.zeros(e - a))
            if t is None:
                o, m, l = _attend_blocks(qf, qsr, chunks, vdec, beta_of, hh, 0, nb, sl2, tau, stats, p_round)
                out[a:e, hh] = o * (1.0 / l)[:, None]
                continue
            parts = [_attend_blocks(qf, qsr, chunks, vdec, beta_of, hh, j0, j1, sl2, tau, stats, p_round)
                     for j0, j1 in sched[hh * q_tiles + t]]
            out[a:e, hh] = merge_partials(parts)
    return out


def attention_exact_max(q, chunks, sm_scale=None, q_block=1024):
    """The same scheme with each row's exact max over all keys (two passes): P is rounded against the final
    max instead of the running one. Returns fp32 [Lq, H, D]."""
    q = _as_lhd(q)
    lq, h, d = q.shape
    sl2 = _sl2(sm_scale, d)
    q8, qs = quant_q(q)
    multi = len(chunks) > 1
    vdec = [dequant_v_planes(c) for c in chunks]
    bias = [q_bias(q, c["km"]) * sl2 if multi else None for c in chunks]
    out = torch.empty(lq, h, d, dtype=torch.float32)
    for hh in range(h):
        for a in range(0, lq, q_block):
            e = min(lq, a + q_block)
            qsr = qs[hh].repeat_interleave(Q_GROUP)[a:e]
            logits = []
            for ci, c in enumerate(chunks):
                first, n = c.get("first", 0), c["n"]
                s_int = torch.matmul(q8[hh, a:e].float(), c["k8"][hh, first:first + n].float().t())
                ksr = c["k_scale"][hh].repeat_interleave(K_BLOCK)[first:first + n]
                s = s_int * ((qsr[:, None] * ksr[None, :]) * sl2)
                if multi:
                    s = s + bias[ci][hh, a:e, None]
                logits.append(s)
            m = torch.stack([s.amax(dim=1) for s in logits], 1).amax(dim=1)
            num = torch.zeros(e - a, d, dtype=torch.float32)
            den = torch.zeros(e - a, dtype=torch.float32)
            for ci, c in enumerate(chunks):
                p = torch.exp2(logits[ci] - m[:, None] + P_OFFSET)
                den = den + p.sum(dim=1)
                p8 = e4m3_decode(e4m3_encode(p))
                hi, lo = vdec[ci]
                num = num + torch.matmul(p8, hi[hh, c.get("first", 0):])
                if lo is not None:
                    pl = bf6_round(p / P_LO_SCALE) * P_LO_SCALE
                    num = num + torch.matmul(pl, lo[hh, c.get("first", 0):])
            out[a:e, hh] = num / den[:, None]
    return out


def sdpa_fp32(q, k, v, sm_scale=None):
    """fp32 softmax attention reference, per head: q [Lq, H, D], k/v [Lk, H, D] -> fp32 [Lq, H, D]."""
    q, k, v = _as_lhd(q), _as_lhd(k), _as_lhd(v)
    d = q.shape[-1]
    sm_scale = d ** -0.5 if sm_scale is None else sm_scale
    out = torch.empty(q.shape, dtype=torch.float32)
    for hh in range(q.shape[1]):
        s = torch.matmul(q[:, hh].float(), k[:, hh].float().t()) * sm_scale
        out[:, hh] = torch.matmul(torch.softmax(s, dim=1), v[:, hh].float())
    return out


def merge_partials(parts):
    """Split-KV merge (experiments/bench_attn/splitkv/README.md:62) in the exp2 domain.

    parts: list of (o_unnormalised [Lq, D], m [Lq], d [Lq]), in key order; returns
    O = sum 2^(m_i - M) o_i * (1 / sum 2^(m_i - M) d_i), M = max m_i, summed piece by piece in the given order
    (the merge kernel's order and its multiply by the reciprocal)."""
    m = torch.stack([p[1] for p in parts]).amax(dim=0)
    num = torch.zeros_like(parts[0][0])
    den = torch.zeros_like(parts[0][2])
    for po, pm, pl in parts:
        wgt = torch.exp2(pm - m)
        den = den + wgt * pl
        num = num + wgt[:, None] * po
    return num * (1.0 / den)[:, None]


def make_inputs(lq, lk, h=12, d=HEAD_DIM, seed=0, mem_chunks=0, chunk_len=None):
    """Seeded synthetic inputs in the fixed generation order Q, K, K-offset, V, then per memory chunk K, V.

    Q, V ~ N(0, 1); K ~ N(0, 1) + o[h, d] with o ~ N(0, 3) constant over tokens; memory chunk values
    ~ N(0, 1.5). Tensors are bf16 in NHD [1, L, H, D].
    """
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, lq, h, d, generator=g)
    k = torch.randn(1, lk, h, d, generator=g)
    off = torch.randn(1, 1, h, d, generator=g) * 3.0
    v = torch.randn(1, lk, h, d, generator=g)
    mem = []
    for _ in range(mem_chunks):
        n = chunk_len or lk
        mk = torch.randn(1, n, h, d, generator=g) * 1.5
        mv = torch.randn(1, n, h, d, generator=g) * 1.5
        mem.append((mk.to(torch.bfloat16), mv.to(torch.bfloat16)))
    return q.to(torch.bfloat16), (k + off).to(torch.bfloat16), v.to(torch.bfloat16), mem


def attention_ops(lq, lk, h, d=HEAD_DIM, b=1):
    """Algorithmic ops of one attention call: 4 * B * H * Lq * Lk * d (tools/roofline.py:91-95)."""
    return 4.0 * b * h * lq * lk * d


def requant_bytes(n, h, d=HEAD_DIM, v_planes=1):
    """Bytes of one chunk's re-quant: read bf16 K and V once, write int8 K and `v_planes` e4m3 V planes once,
    plus the per-block K scales and the per-channel mean and V scale (one plane: the algorithmic count)."""
    nb = pad_to(n, K_BLOCK) // K_BLOCK
    return 2 * n * h * d * 2 + (1 + v_planes) * n * h * d + nb * h * 4 + 2 * h * d * 4

