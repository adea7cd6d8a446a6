"""Thin torch-side wrappers over the C-ABI: device memory and the current stream come from torch, the work is
done by the HIP kernels in liblbw_attn.so. Nothing here computes on the CPU."""
import ctypes

import torch

from . import _lib

HEAD_DIM = 128
K_BLOCK = 64
Q_TILE = 256
Q_GROUP = 32
MAX_SEGMENTS = 8
V_TABLE_BYTES = 256   # E8M0 V scales per 64-key block: 2 key groups x 128 channels
V_LO_ROW = 48         # bytes of a channel's 64 bf6 residual codes in a block
ctypes_i32 = ctypes.c_int32


def pad_to(n, m):
    return (n + m - 1) // m * m


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _require_cuda_bf16(name, t):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor (the quantized path has no CPU implementation)")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous head dim of {HEAD_DIM}, got shape {tuple(t.shape)}")


DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1}   # LBW_DTYPE_BF16 / LBW_DTYPE_FP16 of include/lbw_attn.h


def _require_cuda_16(name, t):
    """A device tensor of bf16 or fp16 with a contiguous 128-wide head dim (the quantisers' inputs); returns the
    format code the C-ABI takes."""
    if t.dtype not in DTYPE_CODE:
        raise TypeError(f"{name} must be bfloat16 or float16, got {t.dtype}")
    _require_cuda_bf16(name, t.view(torch.bfloat16) if t.dtype == torch.float16 else t)
    return DTYPE_CODE[t.dtype]


def _same_device(what, *tensors):
    """Every tensor (None skipped) on one device: a kernel launched on the current device would otherwise read or
    write another GPU's memory through a raw pointer."""
    devs = {t.device for t in tensors if t is not None}
    if len(devs) > 1:
        raise ValueError(f"{what}: tensors on different devices {sorted(str(d) for d in devs)}")


class RingCache:
    """Quantised K/V ring for `layers` layers x `slots` chunk slots of capacity `cap` tokens (a multiple of 64).

    Device layout (include/lbw_attn.h): k8 int8 [L, S, BH, cap, 128]; k_scale fp32 [L, S, BH, cap/64];
    km fp32 [L, S, BH, 128]; v8 uint8 [L, S, BH, cap/64, 128, 64] (e4m3); with v_terms=2 the residual plane v8lo
    uint8 [L, S, BH, cap/64, 128, 48] (bf6 codes, 48 bytes per channel and block); v_scale uint8
    [L, S, BH, cap/64, 256], the E8M0 V scales of each 64-key block (byte (32 g + c % 32) * 4 + c / 32 = 127 + e for
    channel c and key group g, the keys 32 g .. 32 g + 31 of the block).
    """

    def __init__(self, layers, batch, heads, cap, slots, device, v_terms=2, zero=True):
        if cap % K_BLOCK:
            raise ValueError("cap must be a multiple of 64")
        if v_terms not in (1, 2):
            raise ValueError("v_terms must be 1 or 2")
        self.layers, self.batch, self.heads, self.cap, self.slots = layers, batch, heads, cap, slots
        bh, nb = batch * heads, cap // K_BLOCK
        dev = torch.device(device)
        # zero=False leaves the memory uninitialised: for a ring whose every attended block is re-quantised before
        # it is read (the drop-in call re-quantises the whole window), clearing it is wasted bandwidth
        new = torch.zeros if zero else torch.empty
        self.k8 = new(layers, slots, bh, cap, HEAD_DIM, dtype=torch.int8, device=dev)
        self.k_scale = new(layers, slots, bh, nb, dtype=torch.float32, device=dev)
        self.km = new(layers, slots, bh, HEAD_DIM, dtype=torch.float32, device=dev)
        self.v_terms = v_terms
        self.v8 = new(layers, slots, bh, nb, HEAD_DIM, K_BLOCK, dtype=torch.uint8, device=dev)
        self.v8lo = new(layers, slots, bh, nb, HEAD_DIM, V_LO_ROW, dtype=torch.uint8, device=dev) \
            if v_terms == 2 else None
        self.v_scale = torch.empty(layers, slots, bh, nb, V_TABLE_BYTES, dtype=torch.uint8, device=dev)
        if zero:
            self.v_scale.fill_(127)   # scale 1
        self.device = dev

    @property
    def bh(self):
        return self.batch * self.heads

    def layer_view(self, layer):
        """(k8, k_scale, km, v8, v8lo or None, v_scale) of one layer, for the per-layer entry points."""
        return (self.k8[layer], self.k_scale[layer], self.km[layer], self.v8[layer],
                self.v8lo[layer] if self.v8lo is not None else None, self.v_scale[layer])


def requant_workspace(layers, bh, length, device):
    nbytes = _lib.load().lbw_kv_requant_workspace_bytes(layers, bh, length)
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def kv_requant(k, v, ring, slot, layer0=0, workspace=None):
    """Quantise bf16 (or fp16) K, V chunks into `slot` of `ring`.

    k, v: [B, L, H, 128] (one layer; written to layer `layer0`) or [layers, B, L, H, 128] (layers
    layer0 .. layer0 + layers - 1), any strides with a contiguous head dim.
    """
    lib = _lib.load()
    dtype = _require_cuda_16("k", k)
    if _require_cuda_16("v", v) != dtype:
        raise TypeError(f"k ({k.dtype}) and v ({v.dtype}) must have one dtype")
    if k.shape != v.shape:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ")
    _same_device("kv_requant", k, v, ring.k8, workspace)
    if k.dim() == 4:
        k, v = k.unsqueeze(0), v.unsqueeze(0)
    nl, b, n, h, _ = k.shape
    if b != ring.batch or h != ring.heads or n > ring.cap or layer0 + nl > ring.layers:
        raise ValueError(f"chunk {tuple(k.shape)} does not fit the ring "
                         f"(layers {ring.layers}, batch {ring.batch}, heads {ring.heads}, cap {ring.cap})")
    if workspace is None:
        workspace = requant_workspace(nl, b * h, n, k.device)
    ks, vs = k.stride(), v.stride()
    st = lib.lbw_kv_requant(
        _ptr(k), _ptr(v), dtype, nl, b, n, h, ks[0], ks[1], ks[2], ks[3], vs[0], vs[1], vs[2], vs[3],
        _ptr(ring.k8[layer0]), _ptr(ring.k_scale[layer0]), _ptr(ring.km[layer0]), _ptr(ring.v8[layer0]),
        _ptr(ring.v8lo[layer0]) if ring.v8lo is not None else None, _ptr(ring.v_scale[layer0]),
        ring.slots, ring.cap, slot, _ptr(workspace), _stream(k))
    _lib.check(st, "lbw_kv_requant")


def quant_q(q, layout="NHD", ring=None, layer=0, seg_slots=()):
    """bf16 / fp16 Q -> (q8 [BH, Lp, 128], q_scale [BH, Lp/32], bias [n_seg, BH, Lp] or None)."""
    lib = _lib.load()
    dtype = _require_cuda_16("q", q)
    b, lq, h, s_b, s_t, s_h = _dims(q, layout)
    if len(seg_slots) > 1:
        _same_device("quant_q", q, ring.km)
    bh, lp = b * h, pad_to(lq, Q_TILE)
    q8 = torch.empty(bh, lp, HEAD_DIM, dtype=torch.int8, device=q.device)
    qs = torch.empty(bh, lp // Q_GROUP, dtype=torch.float32, device=q.device)
    n_seg = len(seg_slots)
    bias = None
    km_ptr, slots, seg_arr = None, 1, None
    if n_seg > 1:
        bias = torch.empty(n_seg, bh, lp, dtype=torch.float32, device=q.device)
        km_ptr, slots = _ptr(ring.km[layer]), ring.slots
        seg_arr = (ctypes_i32 * n_seg)(*seg_slots)
    st = lib.lbw_quant_q(_ptr(q), dtype, b, lq, h, s_b, s_t, s_h, _ptr(q8), _ptr(qs), km_ptr, slots, n_seg,
                         seg_arr, _ptr(bias), _stream(q))
    _lib.check(st, "lbw_quant_q")
    return q8, qs, bias


def _require_rows(name, x, heads):
    """A projection [B, L, heads * 128] bf16 on the device with contiguous channels."""
    if not x.is_cuda:
        raise ValueError(f"{name} must be a device tensor (the quantized path has no CPU implementation)")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {x.dtype}")
    if x.dim() != 3 or x.shape[-1] != heads * HEAD_DIM or x.stride(-1) != 1:
        raise ValueError(f"{name} must be [B, L, {heads * HEAD_DIM}] with contiguous channels, got "
                         f"{tuple(x.shape)} / strides {x.stride()}")


def _require_norm_rope(weight, heads, rope):
    if weight.dtype != torch.bfloat16 or tuple(weight.shape) != (heads * HEAD_DIM,) or not weight.is_contiguous():
        raise ValueError(f"norm weight must be contiguous bf16 ({heads * HEAD_DIM},), got {weight.dtype} "
                         f"{tuple(weight.shape)}")
    t = rope.table
    if t.dtype != torch.float64 or t.dim() != 3 or tuple(t.shape[1:]) != (HEAD_DIM // 2, 2) or not t.is_contiguous():
        raise ValueError(f"rope table must be contiguous float64 [rows, {HEAD_DIM // 2}, 2], got {tuple(t.shape)}")
    if t.device != weight.device:
        raise ValueError("the rope table and the norm weight must be on the projection's device")


def norm_rope_quant_q(q, heads, weight, eps, rope, ring=None, layer=0, seg_slots=(), want_roped=False):
    """The q projection [B, Lq, heads * 128] bf16 -> RMSNorm (weight, eps) -> rotary embedding (`rope`: a
    ChunkRope) -> (q8, q_scale, bias or None, roped bf16 [B, Lq, H, 128] or None), the quantised Q in the layouts
    of quant_q."""
    lib = _lib.load()
    _require_rows("q", q, heads)
    _require_norm_rope(weight, heads, rope)
    _same_device("norm_rope_quant_q", q, weight, rope.table, ring.km if len(seg_slots) > 1 else None)
    b, lq = q.shape[0], q.shape[1]
    bh, lp = b * heads, pad_to(lq, Q_TILE)
    q8 = torch.empty(bh, lp, HEAD_DIM, dtype=torch.int8, device=q.device)
    qs = torch.empty(bh, lp // Q_GROUP, dtype=torch.float32, device=q.device)
    n_seg = len(seg_slots)
    bias, km_ptr, slots, seg_arr = None, None, 1, None
    if n_seg > 1:
        bias = torch.empty(n_seg, bh, lp, dtype=torch.float32, device=q.device)
        km_ptr, slots = _ptr(ring.km[layer]), ring.slots
        seg_arr = (ctypes_i32 * n_seg)(*seg_slots)
    roped = torch.empty(b, lq, heads, HEAD_DIM, dtype=torch.bfloat16, device=q.device) if want_roped else None
    os_ = roped.stride()[:3] if roped is not None else (0, 0, 0)
    st = lib.lbw_norm_rope_quant_q(_ptr(q), b, lq, heads, q.stride(0), q.stride(1), _ptr(weight), float(eps),
                                   _ptr(rope.table), rope.table.shape[0], rope.grid_h, rope.grid_w, rope.start_frame,
                                   _ptr(q8), _ptr(qs), km_ptr, slots, n_seg, seg_arr, _ptr(bias), _ptr(roped),
                                   *os_, _stream(q))
    _lib.check(st, "lbw_norm_rope_quant_q")
    return q8, qs, bias, roped


def norm_rope_kv_requant(k, v, heads, weight, eps, rope, ring, slot, layer=0, k_out=None, workspace=None):
    """The k projection [B, L, heads * 128] bf16 -> RMSNorm -> rotary embedding -> roped bf16 K (into `k_out`,
    [B, L, H, 128], allocated when None), and slot `slot` of `layer` of `ring` re-quantised from it and v
    [B, L, H, 128] exactly as kv_requant would. Returns k_out."""
    lib = _lib.load()
    _require_rows("k", k, heads)
    _require_norm_rope(weight, heads, rope)
    _require_cuda_bf16("v", v)
    b, n = k.shape[0], k.shape[1]
    if tuple(v.shape) != (b, n, heads, HEAD_DIM):
        raise ValueError(f"v {tuple(v.shape)} does not match k {tuple(k.shape)}")
    if b != ring.batch or heads != ring.heads or n > ring.cap or not 0 <= layer < ring.layers:
        raise ValueError(f"chunk of {n} tokens does not fit the ring (batch {ring.batch}, heads {ring.heads}, "
                         f"cap {ring.cap}, layers {ring.layers})")
    if k_out is None:
        k_out = torch.empty(b, n, heads, HEAD_DIM, dtype=torch.bfloat16, device=k.device)
    _require_cuda_bf16("k_out", k_out)
    _same_device("norm_rope_kv_requant", k, v, weight, rope.table, ring.k8, k_out, workspace)
    if tuple(k_out.shape) != (b, n, heads, HEAD_DIM):
        raise ValueError(f"k_out {tuple(k_out.shape)} must be {(b, n, heads, HEAD_DIM)}")
    if workspace is None:
        workspace = requant_workspace(1, b * heads, n, k.device)
    k8, ksc, km, v8, v8lo, vsc = ring.layer_view(layer)
    vs, os_ = v.stride(), k_out.stride()
    st = lib.lbw_norm_rope_kv_requant(_ptr(k), _ptr(v), b, n, heads, k.stride(0), k.stride(1), vs[0], vs[1], vs[2],
                                      _ptr(weight), float(eps), _ptr(rope.table), rope.table.shape[0], rope.grid_h,
                                      rope.grid_w, rope.start_frame, _ptr(k_out), os_[0], os_[1], os_[2], _ptr(k8),
                                      _ptr(ksc), _ptr(km), _ptr(v8), _ptr(v8lo), _ptr(vsc), ring.slots, ring.cap,
                                      slot, _ptr(workspace), _stream(k))
    _lib.check(st, "lbw_norm_rope_kv_requant")
    return k_out


class CrossContext:
    """One layer's cross-attention context in the kernel's layout: K [BH, Lkp, 128] and V^T [BH, 128, Lkp] bf16
    (Lkp = ceil64(Lk), padding zero), made once from k, v [B, Lk, H, 128] (lbw_cross_prepare)."""

    def __init__(self, k, v):
        lib = _lib.load()
        _require_cuda_bf16("k", k)
        _require_cuda_bf16("v", v)
        if k.dim() != 4 or tuple(v.shape) != tuple(k.shape):
            raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must be the same [B, Lk, H, 128]")
        _same_device("CrossContext", k, v)
        b, lk, h, _ = k.shape
        lkp = pad_to(lk, K_BLOCK)
        self.batch, self.lk, self.heads = b, lk, h
        self.k = torch.empty(b * h, lkp, HEAD_DIM, dtype=torch.bfloat16, device=k.device)
        self.vt = torch.empty(b * h, HEAD_DIM, lkp, dtype=torch.bfloat16, device=k.device)
        ks, vs = k.stride(), v.stride()
        st = lib.lbw_cross_prepare(_ptr(k), _ptr(v), b, lk, h, ks[0], ks[1], ks[2], vs[0], vs[1], vs[2],
                                   _ptr(self.k), _ptr(self.vt), _stream(k))
        _lib.check(st, "lbw_cross_prepare")


def cross_attn_fwd(q, ctx, out=None, sm_scale=None, k_lens=None):
    """Cross-attention of q [B, Lq, H, 128] bf16 against a CrossContext; k_lens: None or B key counts (host
    ints). Returns out [B, Lq, H, 128] bf16."""
    lib = _lib.load()
    _require_cuda_bf16("q", q)
    b, lq, h, _ = q.shape
    if (b, h) != (ctx.batch, ctx.heads):
        raise ValueError(f"q {tuple(q.shape)} does not match the context (batch {ctx.batch}, heads {ctx.heads})")
    if out is None:
        out = torch.empty_like(q)
    _require_cuda_bf16("out", out)
    if tuple(out.shape) != tuple(q.shape):
        raise ValueError(f"out {tuple(out.shape)} must be {tuple(q.shape)}")
    _same_device("cross_attn_fwd", q, ctx.k, out)
    lens = None
    if k_lens is not None:
        vals = [int(x) for x in (k_lens.tolist() if hasattr(k_lens, "tolist") else k_lens)]
        if len(vals) != b:
            raise ValueError(f"k_lens needs {b} entries, got {len(vals)}")
        lens = (ctypes_i32 * b)(*vals)
    sm_scale = HEAD_DIM ** -0.5 if sm_scale is None else float(sm_scale)
    qs, os_ = q.stride(), out.stride()
    st = lib.lbw_cross_attn_fwd(_ptr(q), b, lq, h, qs[0], qs[1], qs[2], _ptr(ctx.k), _ptr(ctx.vt), ctx.lk, lens,
                                _ptr(out), os_[0], os_[1], os_[2], sm_scale, _stream(q))
    _lib.check(st, "lbw_cross_attn_fwd")
    return out


def quant_rows_fp8(x):
    """Rowwise e4m3 of a 2-d bf16 / fp32 device tensor x [rows, cols] (cols a multiple of 16, unit column stride):
    (x8 float8_e4m3fn [rows, cols], scale fp32 [rows, 1]) with x ~ x8 * scale."""
    lib = _lib.load()
    if not x.is_cuda:
        raise ValueError("x must be a device tensor (the FP8 path has no CPU implementation)")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x must be bfloat16 or float32, got {x.dtype}")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError(f"x must be 2-d with contiguous rows, got {tuple(x.shape)} / {x.stride()}")
    rows, cols = x.shape
    x8 = torch.empty(rows, cols, dtype=torch.float8_e4m3fn, device=x.device)
    scale = torch.empty(rows, 1, dtype=torch.float32, device=x.device)
    st = lib.lbw_quant_rows_fp8(_ptr(x), int(x.dtype == torch.float32), rows, cols, x.stride(0), _ptr(x8),
                                _ptr(scale), _stream(x))
    _lib.check(st, "lbw_quant_rows_fp8")
    return x8, scale


def quant_rows_fp8_gelu(x):
    """GELU (tanh form, rounded to bf16) of a 2-d bf16 device tensor x [rows, cols], then its rowwise e4m3 as
    quant_rows_fp8 gives it, in one pass (lbw_quant_rows_fp8_gelu): (x8 float8_e4m3fn [rows, cols], scale fp32
    [rows, 1]) with gelu(x) ~ x8 * scale."""
    lib = _lib.load()
    if not x.is_cuda:
        raise ValueError("x must be a device tensor (the FP8 path has no CPU implementation)")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16, got {x.dtype}")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError(f"x must be 2-d with contiguous rows, got {tuple(x.shape)} / {x.stride()}")
    rows, cols = x.shape
    x8 = torch.empty(rows, cols, dtype=torch.float8_e4m3fn, device=x.device)
    scale = torch.empty(rows, 1, dtype=torch.float32, device=x.device)
    st = lib.lbw_quant_rows_fp8_gelu(_ptr(x), rows, cols, x.stride(0), _ptr(x8), _ptr(scale), _stream(x))
    _lib.check(st, "lbw_quant_rows_fp8_gelu")
    return x8, scale


def quant_mx_fp8(x, rows_pad=None):
    """MXFP8 of a 2-d bf16 / fp32 device tensor x [rows, cols] (cols a multiple of 32, unit column stride):
    (x8 float8_e4m3fn [rows_pad, cols], scale float8_e8m0fnu [rows_pad, cols / 32]), one power-of-two scale per 32
    values; rows past `rows` (up to rows_pad, default rows) are zero with scale 1."""
    lib = _lib.load()
    if not x.is_cuda:
        raise ValueError("x must be a device tensor (the FP8 path has no CPU implementation)")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x must be bfloat16 or float32, got {x.dtype}")
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError(f"x must be 2-d with contiguous rows, got {tuple(x.shape)} / {x.stride()}")
    rows, cols = x.shape
    rows_pad = rows if rows_pad is None else int(rows_pad)
    x8 = torch.empty(rows_pad, cols, dtype=torch.float8_e4m3fn, device=x.device)
    e8 = torch.empty(rows_pad, cols // 32, dtype=torch.uint8, device=x.device)
    st = lib.lbw_quant_mx_fp8(_ptr(x), int(x.dtype == torch.float32), rows, rows_pad, cols, x.stride(0), _ptr(x8),
                              _ptr(e8), _stream(x))
    _lib.check(st, "lbw_quant_mx_fp8")
    return x8, e8.view(torch.float8_e8m0fnu)


_ATTN_WS = {}


def attn_workspace(device, stream=None):
    """The attention's scratch (partials of split query tiles) for `device` and the stream the call is launched
    on, allocated once per (device, stream): calls on different streams may run at the same time, and calls that
    share a workspace must not overlap."""
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if stream is None:
        stream = torch.cuda.current_stream(idx).cuda_stream
    key = (dev.type, idx, stream)
    if key not in _ATTN_WS:
        nbytes = _lib.load().lbw_attn_workspace_bytes()
        _ATTN_WS[key] = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=torch.device(dev.type, idx))
    return _ATTN_WS[key]


def key_blocks(seg_lens, seg_firsts=None):
    """64-key blocks the attention walks over chunks read over [first, first + len) of their slots."""
    firsts = seg_firsts or [0] * len(seg_lens)
    return sum((f % K_BLOCK + n + K_BLOCK - 1) // K_BLOCK for f, n in zip(firsts, seg_lens))


def attn_fwd(q8, q_scale, bias, batch, lq, heads, ring, layer, seg_slots, seg_lens, out, layout="NHD",
             sm_scale=None, workspace=None, noalloc=False, seg_firsts=None, logits=None):
    """Quantized attention of quantised Q over the chunks `seg_slots` of one layer of `ring`, chunk c read over
    tokens [seg_firsts[c], seg_firsts[c] + seg_lens[c]) of its slot (seg_firsts None: from token 0), written into
    bf16 `out` ([B, Lq, H, 128] NHD or [B, H, Lq, 128] HND). noalloc=True calls lbw_attn_fwd_noalloc, whose scratch
    is the library's fixed per-GPU array (no workspace). logits: an int32 [BH, Lp, 64 * key_blocks] tensor makes
    the call run the kernel's checking build (lbw_qk_logits_i32), which also writes each block's raw QK^T
    accumulator words there."""
    lib = _lib.load()
    n_seg = len(seg_slots)
    if not 1 <= n_seg <= MAX_SEGMENTS or len(seg_lens) != n_seg:
        raise ValueError(f"need 1..{MAX_SEGMENTS} chunks with a length each, got {seg_slots} / {seg_lens}")
    if seg_firsts is not None and len(seg_firsts) != n_seg:
        raise ValueError(f"need a first token per chunk, got {seg_firsts} for {n_seg} chunks")
    if any(int(n) < 1 for n in seg_lens) or any(int(f) < 0 or int(f) + int(n) > ring.cap for f, n in
                                                zip(seg_firsts or [0] * n_seg, seg_lens)):
        raise ValueError(f"chunk ranges (first {seg_firsts}, length {seg_lens}) must lie in slots of {ring.cap}")
    _require_cuda_bf16("out", out)
    _same_device("attn_fwd", q8, q_scale, bias, out, ring.k8, workspace)
    ob, ol, oh, o_b, o_t, o_h = _dims(out, layout)
    if (ob, ol, oh) != (batch, lq, heads):   # the kernel writes every row of this shape through out's strides
        raise ValueError(f"out {tuple(out.shape)} ({layout}) does not hold batch {batch} x {lq} rows x {heads} heads")
    bh, lp = batch * heads, pad_to(lq, Q_TILE)
    # the kernel strides q8, q_scale and bias by the padded row count of *this* lq: buffers quantised for another
    # length would be read past their end or row-shifted
    if (q8.dtype != torch.int8 or tuple(q8.shape) != (bh, lp, HEAD_DIM) or not q8.is_contiguous()
            or q_scale.dtype != torch.float32 or tuple(q_scale.shape) != (bh, lp // Q_GROUP)
            or not q_scale.is_contiguous()):
        raise ValueError(f"q8 {tuple(q8.shape)} / q_scale {tuple(q_scale.shape)} must be contiguous int8 "
                         f"({bh}, {lp}, {HEAD_DIM}) / fp32 ({bh}, {lp // Q_GROUP}) for batch {batch}, heads {heads}, "
                         f"lq {lq}")
    if n_seg == 1:
        if bias is not None:
            raise ValueError("one chunk needs no logit bias: pass bias=None")
    elif (bias is None or bias.dtype != torch.float32 or tuple(bias.shape) != (n_seg, bh, lp)
          or not bias.is_contiguous()):
        raise ValueError(f"{n_seg} chunks need a contiguous fp32 bias ({n_seg}, {bh}, {lp}), got "
                         f"{None if bias is None else tuple(bias.shape)}")
    sm_scale = HEAD_DIM ** -0.5 if sm_scale is None else float(sm_scale)
    k8, ksc, _, v8, v8lo, vsc = ring.layer_view(layer)
    slot_arr = (ctypes_i32 * n_seg)(*seg_slots)
    len_arr = (ctypes_i32 * n_seg)(*seg_lens)
    first_arr = (ctypes_i32 * n_seg)(*seg_firsts) if seg_firsts is not None else None
    if noalloc:
        if logits is not None:
            raise ValueError("the checking build runs through lbw_qk_logits_i32, which takes a workspace")
        st = lib.lbw_attn_fwd_noalloc(_ptr(q8), _ptr(q_scale), _ptr(bias), batch, lq, heads, _ptr(k8), _ptr(ksc),
                                      _ptr(v8), _ptr(v8lo), _ptr(vsc), ring.slots, ring.cap, n_seg, slot_arr, len_arr,
                                      first_arr, _ptr(out), o_b, o_t, o_h, sm_scale, _stream(q8))
        _lib.check(st, "lbw_attn_fwd_noalloc")
        return out
    if workspace is None:
        workspace = attn_workspace(q8.device, _stream(q8))
    if logits is not None:
        want = (bh, lp, K_BLOCK * key_blocks(seg_lens, seg_firsts))
        if logits.dtype != torch.int32 or tuple(logits.shape) != want or not logits.is_contiguous():
            raise ValueError(f"logits must be contiguous int32 {want}, got {logits.dtype} {tuple(logits.shape)}")
        _same_device("qk_logits", q8, logits)
        st = lib.lbw_qk_logits_i32(_ptr(q8), _ptr(q_scale), _ptr(bias), batch, lq, heads, _ptr(k8), _ptr(ksc),
                                   _ptr(v8), _ptr(v8lo), _ptr(vsc), ring.slots, ring.cap, n_seg, slot_arr, len_arr,
                                   first_arr, _ptr(out), o_b, o_t, o_h, sm_scale, _ptr(logits), _ptr(workspace),
                                   _stream(q8))
        _lib.check(st, "lbw_qk_logits_i32")
        return out
    st = lib.lbw_attn_fwd(_ptr(q8), _ptr(q_scale), _ptr(bias), batch, lq, heads, _ptr(k8), _ptr(ksc),
                          _ptr(v8), _ptr(v8lo), _ptr(vsc), ring.slots, ring.cap, n_seg, slot_arr, len_arr, first_arr,
                          _ptr(out), o_b, o_t, o_h, sm_scale, _ptr(workspace), _stream(q8))
    _lib.check(st, "lbw_attn_fwd")
    return out


# S_MAGIC: the bits of 1 / (2 pi), where the attention kernel's int32 QK^T accumulators start
S_MAGIC = 0x3E22F983


def qk_logits(q8, q_scale, bias, batch, lq, heads, ring, layer, seg_slots, seg_lens, seg_firsts=None,
              sm_scale=None):
    """Debug: the attention call of attn_fwd run by the kernel's checking build, returning (raw, out): raw is
    int32 [BH, Lp, 64 * key_blocks] holding every key block's QK^T accumulator words S_MAGIC + q8 . k8 (blocks
    in call order, each the 64 keys of a slot block), out the attention output [B, Lq, H, 128] bf16."""
    bh, lp = batch * heads, pad_to(lq, Q_TILE)
    raw = torch.empty(bh, lp, K_BLOCK * key_blocks(seg_lens, seg_firsts), dtype=torch.int32, device=q8.device)
    out = torch.empty(batch, lq, heads, HEAD_DIM, dtype=torch.bfloat16, device=q8.device)
    attn_fwd(q8, q_scale, bias, batch, lq, heads, ring, layer, seg_slots, seg_lens, out, "NHD", sm_scale,
             seg_firsts=seg_firsts, logits=raw)
    return raw, out


def _dims(x, layout):
    """(B, L, H, stride_batch, stride_tok, stride_head) of an NHD [B, L, H, D] or HND [B, H, L, D] tensor."""
    if x.dim() != 4:
        raise ValueError(f"expected a 4-d tensor, got shape {tuple(x.shape)}")
    s = x.stride()
    if layout == "NHD":
        return x.shape[0], x.shape[1], x.shape[2], s[0], s[1], s[2]
    if layout == "HND":
        return x.shape[0], x.shape[2], x.shape[1], s[0], s[2], s[1]
    raise ValueError(f"tensor_layout must be 'NHD' or 'HND', got {layout!r}")

