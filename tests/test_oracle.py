"""Pins of the CPU oracle (oracle/emu.py) against the mathematics that fixes it: an independent e4m3 encoder
written from the format definition, round-half-even ties, closed forms, exact invariances, int64 brute force,
fp32 softmax attention, and the split-KV merge identity. No GPU needed."""
import math

import numpy as np
import pytest
import torch

from oracle import emu


# ---------------------------------------------------------------- e4m3 (OCP fn) from the format definition

def e4m3_ref(x):
    """Nearest e4m3fn value bits of a Python float |x| <= 448 (ties to even), by enumerating the 256 codes."""
    best = None
    for code in range(256):
        e, m = (code >> 3) & 15, code & 7
        if e == 15 and m == 7:
            continue                                   # NaN
        mag = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        val = -mag if code & 128 else mag
        d = abs(val - x)
        key = (d, m & 1)                               # nearest, then even mantissa
        if best is None or key < best[0] or (key == best[0] and (code & 128) == (128 if x < 0 else 0)):
            best = (key, code, val)
    code = best[1]
    if best[2] == 0.0:                                 # signed zero follows the input's sign
        code = 128 if math.copysign(1.0, x) < 0 else 0
    return code


def test_e4m3_encoder_matches_format_definition():
    rng = np.random.default_rng(0)
    xs = [0.0, -0.0, 448.0, -448.0, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -9, 3 * 2.0 ** -10, 232.0, 240.0, 17.0,
          0.0174, 1.0625, 1.1875, -3.25]
    # every e4m3 value and the midpoints between neighbours (the ties), plus random values
    vals = sorted({emu.e4m3_decode(torch.tensor([c], dtype=torch.uint8)).item() for c in range(256)
                   if (c & 0x7F) != 0x7F})
    xs += vals + [(a + b) / 2 for a, b in zip(vals, vals[1:])]
    xs += list(rng.uniform(-448, 448, 300)) + list(rng.uniform(-0.05, 0.05, 300))
    x32 = torch.tensor(xs, dtype=torch.float32)
    got = emu.e4m3_encode(x32).tolist()
    want = [e4m3_ref(float(v)) for v in x32.tolist()]
    assert got == want


def bf6_ref(x):
    """Nearest bf6 (OCP e3m2, bias 3, no inf / NaN) code of a Python float by enumerating the 64 codes: ties to the
    even mantissa, magnitudes beyond 28 saturating, a value that rounds to zero keeping its sign."""
    if math.isnan(x):
        return 0x1F | (0x20 if math.copysign(1.0, x) < 0 else 0)
    best, a = None, min(abs(x), 28.0)                   # 28 is the largest magnitude
    for code in range(32):
        e, m = (code >> 2) & 7, code & 3
        mag = (m / 4.0) * 2.0 ** -2 if e == 0 else (1 + m / 4.0) * 2.0 ** (e - 3)
        key = (abs(mag - a), m & 1)
        if best is None or key < best[0]:
            best = (key, code)
    return best[1] | (0x20 if math.copysign(1.0, x) < 0 else 0)


def test_bf6_encoder_matches_format_definition():
    """bf6_encode against the enumeration above over every value, every midpoint (the ties), values past the
    range and random ones; and against the codes gfx950's v_cvt_scalef32_2xpk16_bf6_f32 gave for special inputs
    (scale 1): NaN and infinities saturate to 28 with their sign, 26 ties to 24, 0.03125 to +0."""
    vals = sorted({float(emu.bf6_decode(torch.tensor([c], dtype=torch.uint8))) for c in range(64)})
    xs = vals + [(a + b) / 2 for a, b in zip(vals, vals[1:])] + [30.0, -31.99, 1e30, 0.03124, 0.03126, -1e-40]
    xs += list(np.random.default_rng(9).uniform(-30, 30, 400)) + list(np.random.default_rng(10).uniform(-0.3, 0.3, 200))
    x32 = torch.tensor(xs, dtype=torch.float32)
    assert emu.bf6_encode(x32).tolist() == [bf6_ref(float(v)) for v in x32.tolist()]
    codes = torch.arange(64, dtype=torch.uint8)
    assert torch.equal(emu.bf6_encode(emu.bf6_decode(codes)), codes)
    special = torch.tensor([float("nan"), float("inf"), -float("inf"), 28.0, 32.0, -0.0, 0.03125, 0.09375, 26.0,
                            18.0, 7.5, 3.75, 0.21875, -16.0])
    special[0] = -special[0]                              # a negative NaN
    assert emu.bf6_encode(special).tolist() == [0x3F, 0x1F, 0x3F, 0x1F, 0x1F, 0x20, 0x00, 0x02, 0x1E, 0x1C, 0x18,
                                                 0x14, 0x04, 0x3C]


def test_bf6_round_equals_encode_decode():
    """bf6_round (the attention emulation's fast path) against bf6_decode(bf6_encode(x)): every value, every midpoint
    and its float neighbours, random values in and past the range, signed zeros."""
    vals = sorted({float(emu.bf6_decode(torch.tensor([c], dtype=torch.uint8))) for c in range(64)})
    x = torch.tensor(vals + [(a + b) / 2 for a, b in zip(vals, vals[1:])], dtype=torch.float32)
    g = torch.Generator().manual_seed(12)
    x = torch.cat([x, torch.nextafter(x, torch.tensor(100.0)), torch.nextafter(x, torch.tensor(-100.0)),
                   (torch.rand(50000, generator=g) - 0.2) * 40, torch.rand(20000, generator=g) * 0.5,
                   torch.tensor([29.0, 30.0, 31.9, 1e9, -0.0, 0.0, -1e-30])])
    a, b = emu.bf6_round(x), emu.bf6_decode(emu.bf6_encode(x))
    assert torch.equal(a, b) and torch.equal(torch.signbit(a), torch.signbit(b))


def test_bf6_rows_pack_and_unpack():
    codes = torch.randint(0, 64, (2, 3, 128, 64), dtype=torch.uint8, generator=torch.Generator().manual_seed(8))
    rows = emu.pack_bf6_rows(codes)
    assert rows.shape == (2, 3, 128, 48) and torch.equal(emu.unpack_bf6_rows(rows), codes)


# ---------------------------------------------------------------- int8 quantisers

def test_int8_group_quant_closed_form():
    torch.manual_seed(1)
    lq, h = 200, 3
    # rows of group g scaled by 2^g so a wrong row -> group map changes the scales
    q = torch.randn(lq, h, 128) * (2.0 ** (torch.arange(lq) // 32).float())[:, None, None]
    q = q.to(torch.bfloat16)
    q8, qs = emu.quant_q(q)
    assert q8.shape == (h, emu.pad_to(lq, emu.Q_TILE), 128) and qs.shape == (h, emu.pad_to(lq, emu.Q_TILE) // 32)
    x = torch.zeros(h, q8.shape[1], 128)
    x[:, :lq] = q.float().permute(1, 0, 2)
    for hh in range(h):
        for gi in range(qs.shape[1]):
            blk = x[hh, 32 * gi:32 * gi + 32]
            amax = max(float(blk.abs().max()), 1e-7)
            assert qs[hh, gi].item() == np.float32(np.float32(amax) / np.float32(127.0))
            qi = q8[hh, 32 * gi:32 * gi + 32].float()
            assert qi.abs().max() <= 127
            if amax > 1e-7:
                assert qi.abs().max() == 127                          # the largest element maps to +-127
                # within half a step (plus the rounding of 127/amax), checked in fp64
                err = (qi.double() * qs[hh, gi].double() - blk.double()).abs().max().item()
                assert err <= qs[hh, gi].item() * 0.5 * (1 + 1e-5)
    assert torch.all(q8[:, lq:] == 0)                                 # padded rows are zero


def test_int8_round_half_even_ties_and_zero_group():
    # amax = 127 -> recip = 1, so the quantised value is the rounded input itself
    row = torch.zeros(32, 1, 128)
    row[0, 0, 0] = 127.0
    row[1, 0, :8] = torch.tensor([2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5])
    q8, qs = emu.quant_q(row.to(torch.bfloat16))
    assert qs[0, 0].item() == pytest.approx(1.0)
    assert q8[0, 1, :8].tolist() == [2, 4, -2, -4, 0, 0, 2, 126]
    assert torch.all(q8[0, 32:] == 0) and qs[0, 1].item() == np.float32(np.float32(1e-7) / np.float32(127))


def test_last_group_counts_padding_as_zero():
    # Lq = 33: group 1 holds one real row; its scale comes from that row alone
    q = torch.zeros(33, 1, 128)
    q[:32] = 100.0
    q[32, 0, 5] = -3.0
    q8, qs = emu.quant_q(q.to(torch.bfloat16))
    assert qs[0, 1].item() == np.float32(np.float32(3.0) / np.float32(127))
    assert q8[0, 32, 5].item() == -127


# ---------------------------------------------------------------- K mean (fixed order) and smoothing

def mean_by_loops(k):
    """The documented mean order, restated with scalar fp32 loops (tiny inputs only): 4-token sums, eight of them
    per 32-token half left to right, the two halves added, the blocks of each 4-block super-block left to right,
    the super-blocks left to right, then / n. Returns the fp32 mean (before any rounding)."""
    n, h, d = k.shape
    nb = (n + 63) // 64
    out = np.zeros((h, d), dtype=np.float32)
    x = np.zeros((nb * 64, h, d), dtype=np.float32)
    x[:n] = k.float().numpy()
    for hh in range(h):
        for c in range(d):
            tot = np.float32(0)
            for u in range(0, nb, 4):
                sup = np.float32(0)
                for b in range(u, min(nb, u + 4)):
                    halves = []
                    for i in range(2):
                        half = np.float32(0)
                        for q in range(8 * i, 8 * i + 8):
                            s = np.float32(0)
                            for j in range(4):
                                s = np.float32(s + x[64 * b + 4 * q + j, hh, c])
                            half = np.float32(half + s)
                        halves.append(half)
                    sup = np.float32(sup + np.float32(halves[0] + halves[1]))
                tot = np.float32(tot + sup)
            out[hh, c] = np.float32(tot / np.float32(n))
    return torch.from_numpy(out)


@pytest.mark.parametrize("dtype,mant", [(torch.bfloat16, 7), (torch.float16, 10)])
def test_chunk_mean_order_and_accuracy(dtype, mant):
    """The fp32 mean bit for bit against the scalar-loop restatement of the documented order (values with many
    mantissa bits, so a different order would round differently), and the rounded mean within one ulp of the
    input format (bf16, fp16) of the fp64 mean."""
    torch.manual_seed(2)
    scale = torch.tensor([1e3, -7.0, 0.01, 50.0]) if dtype == torch.bfloat16 else torch.tensor([300.0, -7.0, 0.01, 50.0])
    k = (torch.randn(700, 2, 4) * 3 + scale).to(dtype)
    assert torch.equal(emu.chunk_mean(k, rounded=False), mean_by_loops(k))
    km = emu.chunk_mean(k)
    assert torch.equal(km, mean_by_loops(k).to(dtype).float())
    exact = k.double().mean(dim=0)
    ulp = torch.tensor([2.0 ** (math.floor(math.log2(abs(v))) - mant) for v in exact.flatten().tolist()]).view(2, 4)
    assert torch.all((km.double() - exact).abs() <= ulp)              # within one ulp of the true mean


def test_smoothing_makes_k8_invariant_to_channel_offsets():
    # zero-mean noise on a 1/4 grid keeps every fp32 partial sum exact, so the mean is exactly the offset and
    # K - mean is exactly the noise: the int8 K and its scales cannot depend on the offset
    rng = np.random.default_rng(3)
    noise = rng.integers(-16, 17, size=(64, 2, 128)).astype(np.float32) / 4
    noise = np.concatenate([noise, -noise])                          # 128 tokens, column sums exactly 0
    outs = []
    for off in (0.0, 5.5, -24.75):
        k = torch.from_numpy(noise + np.float32(off)).to(torch.bfloat16)
        km = emu.chunk_mean(k)
        assert torch.all(km == off)
        outs.append(emu.quant_k(k, km))
    for k8, ks in outs[1:]:
        assert torch.equal(k8, outs[0][0]) and torch.equal(ks, outs[0][1])


# ---------------------------------------------------------------- V planes and layout

def test_v_scale_power_of_two_edges():
    """The exponent rule at the binade edges: amax exactly 448 * 2^e keeps e; one bf16 step above moves to e + 1;
    an all-zero group uses the 1e-7 floor."""
    vals = torch.tensor([448.0, 450.0, 224.0, 225.0, 1.0, 3.5, 0.0])   # 450: the bf16 value after 448
    v = torch.zeros(64, 1, len(vals))
    v[1, 0] = vals                                                     # key 1 is in group 0; group 1 stays zero
    e = emu.v_group_exponents(v.to(torch.bfloat16))
    assert e.shape == (1, 1, 2, len(vals))
    want = [1.0, 2.0, 0.5, 1.0, 2.0 ** -8, 2.0 ** -7, None]   # 3.5 = 448 * 2^-7 exactly
    for got, w, a in zip(torch.ldexp(torch.ones(len(vals)), e[0, 0, 0]).tolist(), want, vals.tolist()):
        if w is not None:
            assert got == w, (a, got, w)
    for floor_scale in (2.0 ** e[0, 0, 0, -1].item(), 2.0 ** e[0, 0, 1, 0].item()):
        assert 224 < 1e-7 / floor_scale <= 448


def test_v_groups_and_scale_table_layout():
    """Group g is the keys 32 g .. 32 g + 31 of a block: a large value at key 32 (group 1) moves group 1's exponent
    only. The table holds 127 + e[g][c] at byte (32 g + c % 32) * 4 + c // 32 (checked entry by entry), and
    v_exponents_of_table inverts it. The groups are the positions 16 g .. 16 g + 15 and 32 + 16 g .. 32 + 16 g + 15
    of the permuted layout: bytes 16 g .. 16 g + 15 of each lane's PV operand, the MFMA's K-block g."""
    assert emu.V_GROUP_OF_KEY.tolist() == [0] * 32 + [1] * 32
    for g in range(2):
        pos = [int(emu.V_POS_OF_KEY[k]) for k in range(64) if emu.V_GROUP_OF_KEY[k] == g]
        assert sorted(pos) == list(range(16 * g, 16 * g + 16)) + list(range(32 + 16 * g, 48 + 16 * g))
    v = torch.ones(64, 1, 128)
    v[32, 0, 7] = 100.0
    e = emu.v_group_exponents(v.to(torch.bfloat16))
    assert e[0, 0, 1, 7] > e[0, 0, 0, 7] and torch.all(e[0, 0, 0] == e[0, 0, 0, 0])
    assert torch.all(e[0, 0, 1, :7] == e[0, 0, 0, 0]) and torch.all(e[0, 0, 1, 8:] == e[0, 0, 0, 0])
    rng = np.random.default_rng(9)
    e = torch.from_numpy(rng.integers(-40, 40, size=(2, 3, 2, 128)))
    t = emu.v_scale_table(e)
    for hh in range(2):
        for b in range(3):
            for g in range(2):
                for c in range(128):
                    assert int(t[hh, b, (32 * g + c % 32) * 4 + c // 32]) == 127 + int(e[hh, b, g, c])
    assert torch.equal(emu.v_exponents_of_table(t), e)


def test_v_nonfinite_values():
    """A NaN does not enter its group's amax, so the group's other values get the same codes as with a 0 in its
    place, and it becomes a NaN code; an infinity takes its group to exponent 120 (the kernel's bit rule), where its
    finite values underflow to 0 and it becomes a NaN code; the attention output is then NaN in that channel only
    (as the reference's per-channel scale makes the whole channel NaN)."""
    torch.manual_seed(12)
    v = torch.randn(128, 2, 128).to(torch.bfloat16)
    clean = v.clone()
    v[5, 0, 3] = float("nan")
    clean[5, 0, 3] = 0
    v[70, 1, 9] = float("inf")
    a8, alo, at = emu.quant_v(v)
    c8, clo, ct = emu.quant_v(clean)
    pos = int(emu.V_POS_OF_KEY[5])
    nan = (a8 & 0x7F) == 0x7F
    assert bool(nan[0, 0, 3, pos]) and int(nan.sum()) == 2 and bool(nan[1, 1, 9, int(emu.V_POS_OF_KEY[6])])
    keep = torch.ones_like(nan)
    keep[1, 1, 9] = False                              # the infinite value's block and channel
    alo, clo = emu.unpack_bf6_rows(alo), emu.unpack_bf6_rows(clo)
    assert torch.equal(a8[keep & ~nan], c8[keep & ~nan]) and torch.equal(alo[keep & ~nan], clo[keep & ~nan])
    assert bool(((alo[nan] & 0x1F) == 0x1F).all())    # bf6 has no NaN code: the NaN residual saturates to 28
    e = emu.v_exponents_of_table(at)
    assert int(e[1, 1, 0, 9]) == 120 and int(emu.v_exponents_of_table(ct)[1, 1, 0, 9]) != 120
    grp0 = torch.tensor([int(emu.V_POS_OF_KEY[k]) for k in range(32)])   # the infinity's half: keys 0-31
    codes = a8[1, 1, 9, grp0]
    assert int(((codes & 0x7F) == 0x7F).sum()) == 1 and int(((codes & 0x7F) != 0).sum()) == 1   # else +-0
    # through the attention: channel 3 of head 0 is NaN for every query, the rest finite
    q, k, _, _ = emu.make_inputs(40, 128, h=2, seed=3)
    v2 = v.clone()
    v2[70, 1, 9] = 1.0
    out = emu.attention(q, [emu.requant(k, v2)])
    assert bool(out[:, 0, 3].isnan().all()) and int(out.isnan().sum()) == 40


def test_v_position_map_is_a_bijection():
    assert sorted(emu.V_KEY_OF_POS.tolist()) == list(range(64))
    assert np.array_equal(emu.V_POS_OF_KEY[emu.V_KEY_OF_POS], np.arange(64))


def test_v_quant_layout_and_two_term_bound():
    torch.manual_seed(4)
    n, h = 130, 2
    v = (torch.randn(n, h, 128) * torch.rand(1, h, 128) * 4).to(torch.bfloat16)
    v8, v8lo, table = emu.quant_v(v)
    assert v8.shape == (h, 3, 128, 64) and v8lo.shape == (h, 3, 128, 48) and table.shape == (h, 3, 256)
    # each key's scale, from the group amax computed here directly (keys 32 g .. 32 g + 31 of block b)
    vp = torch.zeros(192, h, 128)
    vp[:n] = v.float()
    scale = torch.empty(h, 192, 128)
    for b in range(3):
        for g in range(2):
            keys = [64 * b + k for k in range(32 * g, 32 * g + 32)]
            amax = vp[keys].abs().amax(dim=0).clamp_min(1e-7)                # [h, d]
            s = 2.0 ** torch.ceil(torch.log2(amax.double() / 448)).float()   # the power of two: amax / s in (224, 448]
            assert torch.all(amax / s <= 448) and torch.all(amax / s > 224)
            scale[:, keys] = s[:, None, :]
            e = emu.v_exponents_of_table(table)[:, b, g]
            assert torch.equal(torch.ldexp(torch.ones(h, 128), e), s)
    y = v.float().permute(1, 0, 2) / scale[:, :n]   # [h, n, d], exact
    chunk = {"v8": v8, "v8lo": v8lo, "v_scale": table, "n": n}
    one = emu.dequant_v(chunk, terms=1) / scale[:, :n]
    two = emu.dequant_v(chunk, terms=2) / scale[:, :n]
    # one e4m3 term: half an e4m3 step (2^-4 relative, 2^-10 absolute in the subnormal range)
    tol1 = torch.maximum(y.abs() * 2.0 ** -4, torch.full_like(y, 2.0 ** -10))
    assert torch.all((one - y).abs() <= tol1)
    # two terms: the residual r = y - hi (|r| <= half a step of hi, 2^-4 |y|) carried to bf6 precision: half a bf6
    # step, 2^-3 |r| <= 2^-7 |y| for |r| >= 0.25, and 2^-5 absolute below (bf6's subnormal step is 2^-4)
    tol2 = torch.maximum(y.abs() * 2.0 ** -7, torch.full_like(y, 2.0 ** -5))
    assert torch.all((two - y).abs() <= tol2)
    assert (two - y).abs().mean() < (one - y).abs().mean() / 8
    # the residual row layout, read bit by bit: channel c, position p of V scale group g = (p >> 4) & 1 is code
    # k = (p & 15) + 16 (p >> 5) of the group, at bits 6 k .. 6 k + 5 of its 24 bytes: bytes 0-15 at 16 g of the row,
    # bytes 16-23 at 32 + 8 g (32 + 8 (1 - g) when c & 16)
    hi = emu.e4m3_decode(v8)
    for hh, b, c in ((0, 0, 3), (1, 2, 17), (0, 1, 126), (1, 1, 48)):
        row = [int(x) for x in v8lo[hh, b, c]]
        for p in range(64):
            half, k = (p >> 4) & 1, (p & 15) + 16 * (p >> 5)
            assert int(emu.V_KEY_OF_POS[p]) // 32 == half        # the group of the position is its key's half
            tail = 32 + 8 * (half ^ ((c >> 4) & 1))
            data = row[16 * half:16 * half + 16] + row[tail:tail + 8]
            word = int.from_bytes(bytes(data), "little")
            code = (word >> (6 * k)) & 63
            key = 64 * b + int(emu.V_KEY_OF_POS[p])
            if key < n:
                r = float(y[hh, key, c]) - float(hi[hh, b, c, p])
                assert code == int(emu.bf6_encode(torch.tensor([r]))[0]), (hh, b, c, p)


# ---------------------------------------------------------------- logits

def test_qk_logits_exact_against_int64():
    rng = np.random.default_rng(5)
    q8 = rng.integers(-127, 128, size=(2, 64, 128)).astype(np.int8)
    k8 = rng.integers(-127, 128, size=(2, 96, 128)).astype(np.int8)
    q8[0, 0] = 127
    k8[0, 0] = 127                                                   # |S| at its maximum, 127^2 * 128
    got = emu.qk_logits(torch.from_numpy(q8), torch.from_numpy(k8))
    want = np.einsum("hqd,hkd->hqk", q8.astype(np.int64), k8.astype(np.int64))
    assert got.dtype == torch.int32 and np.array_equal(got.numpy(), want)
    assert want[0, 0, 0] == 127 * 127 * 128


# ---------------------------------------------------------------- attention

def test_attention_within_tolerance_of_fp32_softmax():
    q, k, v, _ = emu.make_inputs(300, 700, h=2, seed=6)
    out = emu.attention(q, [emu.requant(k, v)])
    ref = emu.sdpa_fp32(q, k, v)
    assert (out - ref).abs().max() < 2e-2 and (out - ref).abs().mean() < 2e-3
    # against torch's own SDPA, so the fp32 reference itself is pinned
    qt, kt, vt = (x[0].float().transpose(0, 1) for x in (q, k, v))
    sd = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt).transpose(0, 1)
    assert torch.allclose(ref, sd, atol=1e-5)


def test_attention_invariances():
    q, k, v, _ = emu.make_inputs(128, 320, h=1, seed=7)
    base = emu.attention(q, [emu.requant(k, v)])
    # V scaled by 2: identical V planes, doubled scale -> exactly doubled output
    v2 = (v.float() * 2).to(torch.bfloat16)
    assert torch.equal(emu.attention(q, [emu.requant(k, v2)]), base * 2)
    # keys shifted by a per-channel constant: with column sums exactly zero on a 1/4 grid the mean is exactly
    # the shift, K - mean is exactly the unshifted keys, and (one chunk, no bias) the output is identical
    half = torch.clamp(torch.round(k.float()[:, :160] * 4) / 4, -15, 15)
    kq = torch.cat([half, -half], dim=1).to(torch.bfloat16)
    shift = (torch.arange(128) % 25 - 12).float()                     # integers keep kq + shift bf16-exact
    shifted = (kq.float() + shift).to(torch.bfloat16)
    assert torch.equal(shifted.float() - shift, kq.float())
    a = emu.attention(q, [emu.requant(kq, v)])
    b = emu.attention(q, [emu.requant(shifted, v)])
    assert torch.equal(a, b)


def test_chunked_attention_bias_matches_single_chunk():
    """Splitting the keys into chunks with their own means (bias q . mean_c) computes the same softmax."""
    q, k, v, _ = emu.make_inputs(128, 640, h=1, seed=8)
    one = emu.attention_exact_max(q, [emu.requant(k, v)])
    parts = [emu.requant(k[:, i:i + 160], v[:, i:i + 160]) for i in range(0, 640, 160)]
    four = emu.attention_exact_max(q, parts)
    sd = emu.sdpa_fp32(q, k, v)
    assert (four - sd).abs().mean() < 1.2 * (one - sd).abs().mean()
    assert (four - one).abs().max() < 2e-2


def test_online_and_exact_max_agree():
    """The kernel's online max (lazy rescale) and the exact row max round P to e4m3 at different offsets:
    independent roundings of the same size, so both land equally close to fp32 softmax attention."""
    q, k, v, _ = emu.make_inputs(256, 1000, h=1, seed=9)
    ch = [emu.requant(k, v)]
    sd = emu.sdpa_fp32(q, k, v)
    e_on = (emu.attention(q, ch) - sd).abs()
    e_ex = (emu.attention_exact_max(q, ch) - sd).abs()
    assert 0.8 < e_on.mean() / e_ex.mean() < 1.25
    assert e_on.max() < 2e-2 and e_ex.max() < 2e-2


def test_split_merge_closed_form():
    torch.manual_seed(10)
    s = torch.randn(16, 90, dtype=torch.float64) * 3
    vv = torch.randn(90, 8, dtype=torch.float64)
    ref = torch.softmax(s, dim=1) @ vv
    parts = []
    for a, b in ((0, 31), (31, 64), (64, 90)):
        m = (s[:, a:b] * emu.LOG2E).amax(dim=1)
        p = torch.exp2(s[:, a:b] * emu.LOG2E - m[:, None])
        parts.append((p @ vv[a:b], m, p.sum(dim=1)))
    assert torch.allclose(emu.merge_partials(parts), ref, atol=1e-12)


def test_schedule_covers_every_block_once():
    for n_tiles, nb, gx in ((576, 378, 64), (144, 24, 64), (3, 2, 64), (1, 1, 32), (100, 7, 16)):
        sched = emu.attn_schedule(n_tiles, nb, gx)
        for t in range(n_tiles):
            blocks = [j for j0, j1 in sched[t] for j in range(j0, j1)]
            assert blocks == list(range(nb)), (n_tiles, nb, gx, t)


# ---------------------------------------------------------------- online softmax, chunk switches and split merge

def _ragged_chunks(seed, lens=(200, 150, 333), h=2, lq=300):
    """Chunks with their own K offsets (so the per-chunk means and the logit bias differ) and V amplitudes (so
    the V group scales differ from chunk to chunk)."""
    g = torch.Generator().manual_seed(seed)
    ks, vs = [], []
    for i, n in enumerate(lens):
        ks.append((torch.randn(1, n, h, 128, generator=g) + (2 + i) * torch.randn(1, 1, h, 128, generator=g))
                  .to(torch.bfloat16))
        vs.append((torch.randn(1, n, h, 128, generator=g) * (0.5, 1.0, 3.0)[i % 3]).to(torch.bfloat16))
    q = torch.randn(1, lq, h, 128, generator=g).to(torch.bfloat16)
    return q, ks, vs


def _direct_softmax_fp64(q, chunks, sm_scale=None):
    """Exact softmax attention of the dequantised logits and V in fp64, one row at a time in closed form:
    logit = q8.k8 * q_scale * k_scale + q.km_c (several chunks), base-e softmax, O = sum P V / sum P with V
    dequantised to true units (its group scales applied).
    No block order, no running max, no split: what the online form must equal when P is not rounded."""
    q = q[0]
    lq, h, d = q.shape
    sm = d ** -0.5 if sm_scale is None else sm_scale
    q8, qs = emu.quant_q(q)
    qsr = qs.repeat_interleave(emu.Q_GROUP, dim=1).double()
    out = torch.empty(lq, h, d, dtype=torch.float64)
    for hh in range(h):
        logits, vals = [], []
        for c in chunks:
            a, n = c.get("first", 0), c["n"]
            s = q8[hh, :lq].double() @ c["k8"][hh, a:a + n].double().t()
            s = s * qsr[hh, :lq, None] * c["k_scale"][hh].repeat_interleave(emu.K_BLOCK)[a:a + n].double()[None, :]
            if len(chunks) > 1:
                s = s + (q[:, hh].double() @ c["km"][hh].double())[:, None]
            logits.append(s * sm)
            vals.append(emu.dequant_v(c)[hh, a:a + n].double())
        s = torch.cat(logits, dim=1)
        p = torch.softmax(s, dim=1)
        out[:, hh] = p @ torch.cat(vals, dim=0)
    return out


@pytest.mark.parametrize("gx", [None, 1, 2, 3, 8, 16])
def test_online_split_and_chunk_switch_exact_without_p_rounding(gx):
    """With P unrounded, the oracle's online softmax -- lazy running max, per-chunk bias, O rescaled by the V-scale
    ratio at each chunk switch, tiles cut into pieces and merged -- must equal direct softmax attention of the same
    dequantised logits and V to fp32 rounding. A dropped rescale, bias or merge weight is an O(1) error here."""
    q, ks, vs = _ragged_chunks(31)
    chunks = [emu.requant(k, v) for k, v in zip(ks, vs)]
    want = _direct_softmax_fp64(q, chunks)
    got = emu.attention(q, chunks, schedule_gx=gx, p_round=False).double()
    if gx is not None:   # the schedule really cuts tiles: 4 tiles (2 heads x 2 query tiles) on 8 XCDs
        sched = emu.attn_schedule(4, sum(-(-c["n"] // 64) for c in chunks), gx)
        assert any(len(p) > 1 for p in sched.values()) == (gx > 1)
    err = (got - want).abs().max().item()
    assert err < 2e-5 * want.abs().max().item(), err


def test_row_sum_adds_the_rounded_p():
    """O / l must normalise exactly the weights the hi plane's PV product applies. With V the same in every key
    row (each channel its own value, so every half-block quantises it to the same codes) the output is that row
    whatever the logits, to fp32 rounding, across chunks, a chunk switch and split tiles. The row's values have
    3 mantissa bits, so the scaled y is exact in e4m3 and the residual plane is zero (its product takes P rounded
    to bf6, which the row sum does not normalise exactly). A row sum of the unrounded P would scale the output by
    sum(e4m3(P)) / sum(P), about 1e-3 away from 1 for such weights, which the bound sees."""
    g = torch.Generator().manual_seed(41)
    h, lq = 2, 300
    q = torch.randn(1, lq, h, 128, generator=g).to(torch.bfloat16)
    row = emu.e4m3_decode(emu.e4m3_encode(torch.randn(1, 1, h, 128, generator=g)))
    chunks = []
    for i, n in enumerate((200, 333)):
        k = (torch.randn(1, n, h, 128, generator=g) * (1 + i)).to(torch.bfloat16)
        chunks.append(emu.requant(k, row.expand(1, n, h, 128).to(torch.bfloat16).contiguous()))
    vrow = emu.dequant_v(chunks[0])[:, 0]
    assert torch.equal(vrow, row[0, 0])
    for c in chunks:
        assert torch.equal(emu.dequant_v(c)[:, :c["n"]], vrow[:, None].expand(-1, c["n"], -1))
        assert not emu.unpack_bf6_rows(c["v8lo"]).bitwise_and(0x1F).any()   # the residual plane is all zero
    for gx in (None, 16):
        got = emu.attention(q, chunks, schedule_gx=gx)
        assert ((got - vrow[None]).abs() <= 1e-5 * vrow.abs()[None] + 1e-7).all()
    # the effect a sum of the unrounded weights would have, on weights like these
    p = torch.exp2(torch.rand(533, generator=g) * 8.8)
    assert abs(float(emu.e4m3_decode(emu.e4m3_encode(p)).sum() / p.sum()) - 1) > 1e-4


@pytest.mark.parametrize("gx", [None, 2, 16])
def test_windows_read_from_mid_chunk_exact_without_p_rounding(gx):
    """Chunks read over a window of their keys, as the token window reads them: a suffix from a key inside a
    64-key block (the leading keys of that block masked), a middle range whose first and last keys share one
    block, a suffix from a block boundary, and a whole chunk. With P unrounded the oracle must equal direct
    softmax attention over exactly those keys: a wrong block offset, K-scale index or mask edge is an O(1)
    error for the keys it moves."""
    q, ks, vs = _ragged_chunks(34, lens=(333, 200, 256, 150))
    chunks = [emu.requant(k, v) for k, v in zip(ks, vs)]
    for c, (first, n) in zip(chunks, ((37, 296), (70, 50), (128, 128), (0, 150))):
        c["first"], c["n"] = first, n
    assert [emu.span(c)[2:] for c in chunks] == [(0, 6), (1, 1), (2, 2), (0, 3)]
    want = _direct_softmax_fp64(q, chunks)
    got = emu.attention(q, chunks, schedule_gx=gx, p_round=False).double()
    err = (got - want).abs().max().item()
    assert err < 2e-5 * want.abs().max().item(), err
    # the check can see an off-by-one: the same window shifted by one key moves the direct result past the bound
    moved = [dict(c) for c in chunks]
    moved[0]["first"] = 36
    assert (_direct_softmax_fp64(q, moved) - want).abs().max() > 1e-3


def test_split_pieces_change_only_p_rounding():
    """With P rounded to e4m3, cutting tiles into pieces moves each row's reference max, hence which e4m3 step a
    P lands on: split and unsplit results are two draws of the same rounding noise, equally close to fp32 SDPA
    (a wrong merge would add its own error on top)."""
    q, ks, vs = _ragged_chunks(32)
    chunks = [emu.requant(k, v) for k, v in zip(ks, vs)]
    sd = emu.sdpa_fp32(q, torch.cat(ks, 1), torch.cat(vs, 1))
    base = emu.attention(q, chunks)
    e_base = (base - sd).abs().mean()
    for gx in (2, 8, 16):
        split = emu.attention(q, chunks, schedule_gx=gx)
        assert (split - base).abs().mean() < 1.5 * e_base
        assert 0.75 < (split - sd).abs().mean() / e_base < 1.33


def test_multichunk_within_sdpa_tolerance_of_concatenated_keys():
    """Four chunks with different K means and V amplitudes (per-chunk bias and V-scale ratio rescale), P rounded:
    as close to fp32 SDPA over the concatenated bf16 keys as one chunk over the same keys."""
    q, ks, vs = _ragged_chunks(33, lens=(640, 512, 700, 448), lq=256)
    kk, vv = torch.cat(ks, 1), torch.cat(vs, 1)
    sd = emu.sdpa_fp32(q, kk, vv)
    multi = emu.attention(q, [emu.requant(k, v) for k, v in zip(ks, vs)])
    single = emu.attention(q, [emu.requant(kk, vv)])
    e_m, e_s = (multi - sd).abs(), (single - sd).abs()
    assert e_m.max() < 1.25 * e_s.max()
    assert e_m.mean() < 1.25 * e_s.mean() + 1e-5
