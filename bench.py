"""Benchmark of the quantized DiT attention path on one MI355X.

Workload (one "step"): one chunk-plus-memory attention call at the real chunk shape -- Q [1, 6032, 12, 128]
bf16 against 24128 keys = the current chunk (6032) + 3 cached chunks -- as the DiT layer makes it: quantise
the current chunk's K/V into its ring slot, quantise Q (with the per-chunk logit bias), run the attention
kernel. The cached chunks are quantised from their own bf16 values before the timed region.

Reported (one JSON line on stdout):
  value        attention TOPS of the whole call = 4 * H * Lq * Lk * d / step time, the step replayed as a HIP
               graph (all six launches each replay); eager_ms_per_step is the same step launched from Python
  roofline     the attention call alone (attn_fwd_kernel and the small merge of split query tiles, one
               lbw_attn_fwd): algorithmic ops per call / its HIP-event time vs 5.0 POPS dense INT8/FP8 MFMA
  requant      the K/V re-quant of a saved chunk for 30 layers in one call: algorithmic bytes (bf16 K, V read
               once; int8 K and one e4m3 V plane written once; scales) / time, vs 8 TB/s
  prologue     the fused self-attention prologue per layer call (RMSNorm + RoPE of the q / k projections into
               int8 Q and the current chunk's ring slot): algorithmic bytes / time, vs 8 TB/s
  cross_attention  the DiT's cross-attention per layer call (6032 queries x 512 context tokens, bf16 MFMA):
               algorithmic flops / time, vs 2.5 PFLOP/s dense bf16
  fp8_linear   the DiT's FP8 linears at 6032 tokens (rowwise e4m3 activation quant + hipBLASLt FP8 GEMM):
               flops / time, vs 5.0 PFLOP/s dense fp8
  chunk_sweep  the whole chunk captured in one HIP graph: 30 layers x 5 passes of the step above, then the
               30-layer re-quant that saves the chunk; seconds per chunk
  chunk_sweep_fused  the same chunk as the DiT block runs it from its q / k / v projections: 30 layers x 5
               passes of the fused prologue + attention (causal_self_attention), one HIP graph
  cpu_baseline the torch CPU emulation of the same scheme (oracle/emu.py) on a bounded sample of the call
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

LQ, CHUNK, MEM, H, D = 6032, 6032, 3, 12, 128
LK = CHUNK * (MEM + 1)
LAYERS = 30
MFMA_PEAK_TOPS = 5000.0    # MI355X dense INT8 / FP8 MFMA
HBM_PEAK_GBPS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def synthetic_inputs(lq, lk, h=H, d=D, seed=0, mem_chunks=0, chunk_len=None):
    """Seeded bf16 NHD inputs [1, L, H, D], generated in the order Q, K, K channel offset, V, then K, V of each
    memory chunk: Q, V ~ N(0, 1); K ~ N(0, 1) + o[h, d], o ~ N(0, 3) (the per-channel offset the K mean
    smoothing removes); memory chunks ~ N(0, 1.5)."""
    import torch
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


def attention_ops(lq, lk, h=H, d=D, b=1):
    """Algorithmic ops of one attention call: QK^T and PV, 2 * Lq * Lk * d each per head (one multiply-add =
    2 ops), the count the reference's roofline uses (tools/roofline.py:91-95)."""
    return 4.0 * b * h * lq * lk * d


def requant_bytes(n, h=H, d=D, v_planes=1):
    """Bytes of one chunk's K/V re-quant: bf16 K and V read once; int8 K and `v_planes` e4m3 V planes written
    once; one fp32 scale per 64-token K block; fp32 mean and V scale per (head, channel). With one V plane this
    is the algorithmic count (55,607,760 B per layer at 6032 tokens x 12 heads)."""
    nb = (n + 63) // 64
    return 2 * n * h * d * 2 + (1 + v_planes) * n * h * d + nb * h * 4 + 2 * h * d * 4


def requant_moved_bytes(n, h=H, d=D):
    """Bytes the re-quant's three passes move per layer, as built: bf16 K read twice (statistics, then the
    quantiser: its mean is a reduction over the whole chunk) and V once; int8 K, the e4m3 V plane, its bf6 residual
    plane (0.75 byte a value) and the scale table of every 64-token block written; the K scales and mean; the fp32 K column sums of each 32-token
    half-block written and read back by the finaliser. 83.9 MB per layer at 6032 tokens x 12 heads, 2.52 GB per 30
    layers, 1.1 % below what FETCH_SIZE / WRITE_SIZE count (profiles/hbm_traffic_per_call.md)."""
    nb = (n + 63) // 64
    kv = n * h * d * 2
    return (2 * kv + kv + 2 * nb * 64 * h * d + nb * 64 * h * d * 3 // 4 + nb * h * 256 + nb * h * 4 + h * d * 4 +
            2 * nb * 2 * h * d * 4)


def _profile(name):
    """A counter summary committed in profiles/ (None when absent), with the source fingerprint of the build it
    was measured on (`sources_sha16`, lingbot_world_v2_realtime_amd._lib.sources_sha16)."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f)


def traffic_from_profiles(build):
    """HBM bytes of one attention call (attn_fwd_kernel + merge) measured with rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, scaled by a copy of known size), as committed in profiles/: (bytes, the fingerprint of the build
    they were measured on). The bytes are None unless that build is `build`, the one this run loaded."""
    prof = _profile("attn_fwd_cfg3_traffic.json")
    if prof is None:
        return None, None
    sha = prof.get("sources_sha16")
    return (prof.get("call_hbm_bytes") if sha == build else None), sha


def counters_from_profiles(build):
    """MFMA counters of the attention kernel (rocprofv3 --pmc: SQ_INSTS_VALU_MFMA_MOPS_I8 / _F8 and
    SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE), as committed in profiles/, with the fingerprint of the build
    they were measured on; None unless that build is `build`."""
    prof = _profile("attn_fwd_cfg3_counters.json")
    if prof is None or prof.get("sources_sha16") != build:
        return None
    return prof


def cpu_baseline(heads=3, q_rows=LQ):
    """The torch emulation on a sample: `heads` of the 12 heads, the first `q_rows` queries, all 24128 keys
    (4 chunks), including the Q quantisation and the current chunk's re-quant; scaled to the full call."""
    import torch
    from oracle import emu
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, k, v, mem = synthetic_inputs(LQ, CHUNK, h=heads, seed=0, mem_chunks=MEM, chunk_len=CHUNK)
    chunks = [emu.requant(mk, mv) for mk, mv in mem]
    t0 = time.perf_counter()
    cur = emu.requant(k, v)
    emu.attention(q[:, :q_rows], chunks + [cur])
    dt = time.perf_counter() - t0
    frac = (q_rows / LQ) * heads / H                      # share of the full call's work in the sample
    full_s = dt / frac
    ops = attention_ops(LQ, LK, H, D)
    return {"value": round(ops / full_s / 1e12, 6), "unit": "TOPS", "cores": cores, "kind": "port",
            "sample": f"{heads} of {H} heads x {q_rows} of {LQ} queries x {LK} keys (torch emulation incl. Q and "
                      f"current-chunk quant), {dt:.2f} s, scaled x{1 / frac:.0f} -> {full_s:.1f} s per call"}


def config_table(dev, ms_cfg3, rq_ms, sweep_s, cpu3, heads_cpu=3):
    """The per-config GPU / CPU table: cfg 1 (1508 x 1508) and cfg 2 (6032 x 6032) attention calls on the GPU (one
    chunk, HIP events) and in the CPU emulation (all 12 heads for cfg 1; `heads_cpu` heads scaled for cfg 2); cfg 3
    from the main measurement; cfg 4 (one layer's re-quant) on both; cfg 5 from the graph sweep, its CPU figure
    composed from the measured cfg 3 and cfg 4 CPU times (150 calls + 30 layers)."""
    import torch
    from oracle import emu
    from lingbot_world_v2_realtime_amd import sage_attention
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    out = {}
    for name, n, hs in (("cfg1", 1508, H), ("cfg2", 6032, heads_cpu)):
        q, k, v, _ = synthetic_inputs(n, n, h=H, seed=0)
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
        for _ in range(3):
            sage_attention(qd, kd, vd)
        torch.cuda.synchronize()
        g_ms = _timed(lambda: sage_attention(qd, kd, vd), 20, torch.cuda.current_stream(dev))
        t0 = time.perf_counter()
        chunk = emu.requant(k[:, :, :hs], v[:, :, :hs])
        emu.attention(q[:, :, :hs], [chunk])
        c_s = (time.perf_counter() - t0) * H / hs
        ops = attention_ops(n, n)
        out[name] = {"gpu_ms": round(g_ms, 4), "gpu_TOPS": round(ops / (g_ms * 1e-3) / 1e12, 1),
                     "frac": round(ops / (g_ms * 1e-3) / 1e12 / MFMA_PEAK_TOPS, 4), "cpu_s": round(c_s, 3),
                     "cpu_TOPS": round(ops / c_s / 1e12, 5), "cpu_sample": f"{hs} of {H} heads"}
    ops3 = attention_ops(LQ, LK)
    cpu3_s = ops3 / (cpu3["value"] * 1e12) if cpu3 else None
    out["cfg3"] = {"gpu_ms": round(ms_cfg3, 4), "gpu_TOPS": round(ops3 / (ms_cfg3 * 1e-3) / 1e12, 1),
                   "frac": round(ops3 / (ms_cfg3 * 1e-3) / 1e12 / MFMA_PEAK_TOPS, 4),
                   "cpu_s": None if cpu3_s is None else round(cpu3_s, 2),
                   "cpu_TOPS": None if cpu3 is None else cpu3["value"]}
    q, k, v, _ = synthetic_inputs(CHUNK, CHUNK, h=H, seed=2)
    t0 = time.perf_counter()
    emu.requant(k, v)
    c4 = time.perf_counter() - t0
    b4 = requant_bytes(CHUNK, H, D)
    out["cfg4_layer"] = {"gpu_ms": round(rq_ms / LAYERS, 4), "gpu_GBps": round(b4 / (rq_ms / LAYERS * 1e-3) / 1e9, 1),
                         "cpu_s": round(c4, 3), "cpu_GBps": round(b4 / c4 / 1e9, 3),
                         "note": "GPU: the 30-layer call / 30"}
    out["cfg5_chunk"] = {"gpu_s": sweep_s,
                         "cpu_s": None if cpu3_s is None else round(150 * cpu3_s + LAYERS * c4, 1),
                         "note": "CPU: 150 x the cfg 3 call + 30 x the cfg 4 layer, composed"}
    out["cores"] = cores
    return out


def _timed(fn, n, stream):
    """Mean milliseconds of fn() over n launches, HIP events on `stream`."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(n):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def profile_only(args, dev):
    """One part of the step, alone, for counter runs: the attention call (attn_fwd_kernel + merge) on the
    cfg-3 ring, the 30-layer K/V re-quant, or a plain copy of known size."""
    import torch
    from lingbot_world_v2_realtime_amd import kernels
    from lingbot_world_v2_realtime_amd.layers.kv_quant import QuantKVRing
    stream = torch.cuda.current_stream(dev)
    if args.only == "copy":
        n = 1 << 30                                         # 2^30 bf16 = 2 GiB read + 2 GiB written
        a = torch.empty(n, dtype=torch.bfloat16, device=dev).normal_()
        b = torch.empty_like(a)
        fn = lambda: b.copy_(a)                             # noqa: E731
        nbytes = 2 * a.numel() * a.element_size()
    elif args.only == "prologue":
        ring = QuantKVRing(1, 1, H, CHUNK, slots=MEM + 1, device=dev)
        for _ in range(MEM):
            mk = torch.randn(1, CHUNK, H, D, device=dev).to(torch.bfloat16)
            ring.write(0, mk, mk)
            ring.commit()
        print(json.dumps({"only": "prologue", "result": prologue_call(dev, ring, args.steps, args.warmup)}), flush=True)
        return
    elif args.only == "cross":
        print(json.dumps({"only": "cross", "result": cross_attention_call(dev, args.steps, args.warmup)}), flush=True)
        return
    elif args.only == "requant":
        kl = torch.randn(LAYERS, 1, CHUNK, H, D, device=dev).to(torch.bfloat16)
        vl = torch.randn(LAYERS, 1, CHUNK, H, D, device=dev).to(torch.bfloat16)
        rq = QuantKVRing(LAYERS, 1, H, CHUNK, slots=MEM + 1, device=dev)
        fn = lambda: rq.write_layers(kl, vl)                # noqa: E731
        nbytes = LAYERS * requant_bytes(CHUNK, H, D)
    else:
        q, k, v, mem = synthetic_inputs(LQ, CHUNK, h=H, seed=0, mem_chunks=MEM, chunk_len=CHUNK)
        ring = QuantKVRing(1, 1, H, CHUNK, slots=MEM + 1, device=dev)
        for mk, mv in mem:
            ring.write(0, mk.to(dev), mv.to(dev))
            ring.commit()
        ring.write(0, k.to(dev), v.to(dev))
        slots, lens, _ = ring.attended()
        q = q.to(dev)
        q8, qs, bias = kernels.quant_q(q, "NHD", ring.cache, 0, slots)
        o = torch.empty_like(q)
        fn = lambda: kernels.attn_fwd(q8, qs, bias, 1, LQ, H, ring.cache, 0, slots, lens, o)  # noqa: E731
        nbytes = None
    for _ in range(args.warmup):
        fn()
    torch.cuda.synchronize()
    ms = _timed(fn, args.steps, stream)
    print(json.dumps({"only": args.only, "launches": args.steps, "ms": round(ms, 4), "bytes": nbytes}), flush=True)


def chunk_sweep(dev, layers=LAYERS, passes=5, replays=3):
    """The whole chunk as the causal DiT runs it: `passes` forwards (4 denoising steps and the clean pass) of
    `layers` layers, each layer call re-quantising the current chunk's K/V into its ring slot and attending over
    the current chunk plus 3 cached chunks (Q [1,6032,12,128], 24128 keys), then the 30-layer re-quant that
    saves the chunk -- captured once in a HIP graph and replayed. Returns seconds per chunk and attention TOPS."""
    import torch
    from lingbot_world_v2_realtime_amd.layers.kv_quant import QuantKVRing
    q, k, v, mem = synthetic_inputs(LQ, CHUNK, h=H, seed=1, mem_chunks=MEM, chunk_len=CHUNK)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    ring = QuantKVRing(layers, 1, H, CHUNK, slots=MEM + 1, device=dev)
    for mk, mv in mem:   # the same memory chunks in every layer
        mk, mv = mk.to(dev), mv.to(dev)
        for layer in range(layers):
            ring.write(layer, mk, mv)
        ring.commit()
    del mem
    kl = k.unsqueeze(0).expand(layers, *k.shape)
    vl = v.unsqueeze(0).expand(layers, *v.shape)

    def chunk():
        for _ in range(passes):
            for layer in range(layers):
                ring.write(layer, k, v)
                ring.attend(q, layer)
        ring.write_layers(kl, vl)   # the clean pass's K/V saved for every layer at once

    chunk()                          # warm-up: workspaces and the kernels' first launches
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        chunk()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / replays
    calls = passes * layers
    return {"calls": calls, "layers": layers, "passes": passes, "s_per_chunk": round(sec, 5),
            "attention_TOPS": round(calls * attention_ops(LQ, LK) / sec / 1e12, 1), "hip_graph": True}


def chunk_sweep_fused(dev, layers=LAYERS, passes=5, replays=3):
    """The whole chunk as a DiT block runs it from its projections: `passes` forwards of `layers` layers, each
    layer call the fused self-attention (causal_self_attention: RMSNorm + RoPE of the q / k projections into the
    int8 Q and the current chunk's ring slot, then attention over the chunk + 3 cached chunks, 24128 keys).
    Every forward re-quantises the current slot, so the last (clean) pass is the save and no separate 30-layer
    re-quant follows. Captured once in a HIP graph and replayed; seconds per chunk and attention TOPS."""
    import torch
    from lingbot_world_v2_realtime_amd.layers.kv_quant import QuantKVRing
    from lingbot_world_v2_realtime_amd.layers.prologue import ChunkRope, causal_self_attention, rope_freqs
    g = torch.Generator(device=dev).manual_seed(7)
    ql, kl = (torch.randn(1, CHUNK, H * D, device=dev, generator=g).to(torch.bfloat16) for _ in range(2))
    v = torch.randn(1, CHUNK, H, D, device=dev, generator=g).to(torch.bfloat16)
    wq, wk = ((1 + 0.3 * torch.randn(H * D, device=dev, generator=g)).to(torch.bfloat16) for _ in range(2))
    rope = ChunkRope.for_chunk(rope_freqs(dev), (4, 29, 52), current_start=MEM * CHUNK)
    ring = QuantKVRing(layers, 1, H, CHUNK, slots=MEM + 1, device=dev)
    mk = torch.randn(layers, 1, CHUNK, H, D, device=dev, generator=g).to(torch.bfloat16)
    for _ in range(MEM):
        ring.write_layers(mk, mk)
        ring.commit()
    del mk
    k_out = torch.empty(1, CHUNK, H, D, device=dev, dtype=torch.bfloat16)

    def chunk():
        for _ in range(passes):
            for layer in range(layers):
                causal_self_attention(ring, layer, ql, kl, v, H, wq, wk, rope, k_out=k_out)

    chunk()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        chunk()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / replays
    calls = passes * layers
    return {"calls": calls, "layers": layers, "passes": passes, "s_per_chunk": round(sec, 5),
            "attention_TOPS": round(calls * attention_ops(LQ, LK) / sec / 1e12, 1), "hip_graph": True,
            "per_call": "norm_rope_quant_q + norm_rope_kv_requant (stats, finalise, quant) + attention"}


def prologue_bytes(n=CHUNK, h=H, d=D, n_seg=MEM + 1):
    """Algorithmic bytes of the fused prologue of one layer call: the q and k projections and V read once; the
    int8 Q, int8 K and one e4m3 V plane written once, with their scales, the K mean and the per-chunk logit bias.
    (The roped bf16 K this build writes and the quantiser reads back, and the residual V plane, are overhead.)"""
    lp = (n + 255) // 256 * 256
    nb = (n + 63) // 64
    return 3 * n * h * d * 2 + 3 * n * h * d + h * (lp // 32) * 4 + n_seg * h * lp * 4 + nb * h * 4 + 2 * h * d * 4


def prologue_call(dev, ring, steps=50, warmup=5):
    """The self-attention prologue fused into the quantisation, per layer call at the chunk shape: RMSNorm +
    RoPE of the q projection into int8 Q (+ the 4-chunk logit bias), and of the k projection into the roped K
    and the current chunk's ring slot (lbw_norm_rope_quant_q + lbw_norm_rope_kv_requant), on `ring`'s layer 0."""
    import torch
    from lingbot_world_v2_realtime_amd import kernels
    from lingbot_world_v2_realtime_amd.layers.prologue import ChunkRope, rope_freqs
    g = torch.Generator(device=dev).manual_seed(3)
    ql, kl = (torch.randn(1, CHUNK, H * D, device=dev, generator=g).to(torch.bfloat16) for _ in range(2))
    v = torch.randn(1, CHUNK, H, D, device=dev, generator=g).to(torch.bfloat16)
    wq, wk = (1 + 0.3 * torch.randn(H * D, device=dev, generator=g)).to(torch.bfloat16), \
        (1 + 0.3 * torch.randn(H * D, device=dev, generator=g)).to(torch.bfloat16)
    rope = ChunkRope.for_chunk(rope_freqs(dev), (4, 29, 52), current_start=3 * CHUNK)
    k_out = torch.empty(1, CHUNK, H, D, device=dev, dtype=torch.bfloat16)
    slots, _, _ = ring.attended()
    stream = torch.cuda.current_stream(dev)

    def kpart():
        ring.write_projected(0, kl, v, wk, rope, k_out=k_out)

    def qpart():
        kernels.norm_rope_quant_q(ql, H, wq, 1e-6, rope, ring.cache, 0, slots)

    for _ in range(warmup):
        kpart(), qpart()
    torch.cuda.synchronize()
    k_ms = _timed(kpart, steps, stream)
    q_ms = _timed(qpart, steps, stream)
    nbytes = prologue_bytes()
    ms = k_ms + q_ms
    return {"ms": round(ms, 4), "q_ms": round(q_ms, 4), "kv_ms": round(k_ms, 4), "algorithmic_bytes": nbytes,
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}


BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
CONTEXT = 512               # text context tokens of the cross-attention


def cross_attention_call(dev, steps=50, warmup=5):
    """The DiT's cross-attention per layer call: Q [1,6032,12,128] bf16 against the 512-token text context
    (prepared once per generation), bf16 flash attention on the MFMA with fp32 accumulation (lbw_cross_attn_fwd).
    Algorithmic flops 4 * H * Lq * Lk * d against the dense bf16 peak."""
    import torch
    from lingbot_world_v2_realtime_amd import kernels
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn(1, LQ, H, D, device=dev, generator=g).to(torch.bfloat16)
    k, v = (torch.randn(1, CONTEXT, H, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(2))
    ctx = kernels.CrossContext(k, v)
    out = torch.empty_like(q)
    for _ in range(warmup):
        kernels.cross_attn_fwd(q, ctx, out)
    torch.cuda.synchronize()
    ms = _timed(lambda: kernels.cross_attn_fwd(q, ctx, out), steps, torch.cuda.current_stream(dev))
    flops = attention_ops(LQ, CONTEXT)
    tf = flops / (ms * 1e-3) / 1e12
    return {"lq": LQ, "lk": CONTEXT, "ms": round(ms, 4), "TFLOP/s": round(tf, 1),
            "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), "flops": flops}


FP8_PEAK_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
DIM, FFN = 1536, 8960       # the DiT's model and feed-forward widths


def fp8_linear_calls(dev, steps=30):
    """The DiT's FP8 linears at the chunk shape (6032 tokens): q/k/v/o (1536 -> 1536) and the two feed-forward
    layers (1536 -> 8960, 8960 -> 1536). Per call: the activation quantisation (lbw_quant_rows_fp8) and
    hipBLASLt's rowwise-scaled FP8 GEMM with the bias, timed with hipBLASLt's default solution and with the tuned
    solution table (`ms` is the latter when the table was read). Flops 2 M K N against 5.0 PFLOP/s dense fp8.
    act_quant_call_ms times the quantisation call alone from Python; at ~6-9 us of kernel time it is bound by the
    launch path, so it is an upper bound on the kernel."""
    import torch
    from lingbot_world_v2_realtime_amd import kernels
    import torch.cuda.tunable as tunable
    from lingbot_world_v2_realtime_amd.layers.linear import FP8Linear, use_tuned_gemms
    out = {}
    stream = torch.cuda.current_stream(dev)
    for name, (k, n) in (("proj_1536x1536", (DIM, DIM)), ("ffn_up_1536x8960", (DIM, FFN)),
                         ("ffn_down_8960x1536", (FFN, DIM))):
        lin = torch.nn.Linear(k, n).to(torch.bfloat16).to(dev)
        f = FP8Linear(lin)
        x = torch.randn(1, LQ, k, device=dev).to(torch.bfloat16)
        times = {}
        # hipBLASLt's default solution, then with the tuned-solution table (layers/fp8_gemm_solutions.csv)
        for mode in ("default", "table"):
            table = use_tuned_gemms() if mode == "table" else False
            for _ in range(3):
                f(x)
            torch.cuda.synchronize()
            times[mode] = _timed(lambda: f(x), steps, stream)
            if mode == "table":
                tunable.enable(False)
        ms = times["table"] if table else times["default"]
        q_ms = _timed(lambda: kernels.quant_rows_fp8(x.view(LQ, k)), steps, stream)
        flops = 2.0 * LQ * k * n
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"ms": round(ms, 4), "default_solution_ms": round(times["default"], 4), "gemm_table": table,
                     "act_quant_call_ms": round(q_ms, 4), "TFLOP/s": round(tf, 1),
                     "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4)}
    # the feed-forward block's GELU + down projection: torch's GELU then the FP8 linear (two passes over the
    # 6032 x 8960 activation), against the GELU fused into the activation quantisation (FP8Linear gelu_input,
    # what convert_to_fp8(fuse_gelu=True) builds); both with the tuned solution table
    lin = torch.nn.Linear(FFN, DIM).to(torch.bfloat16).to(dev)
    plain, fused = FP8Linear(lin), FP8Linear(lin, gelu_input=True)
    h = torch.randn(1, LQ, FFN, device=dev).to(torch.bfloat16)
    table = use_tuned_gemms()
    unfused_fn = lambda: plain(torch.nn.functional.gelu(h, approximate="tanh"))   # noqa: E731
    fused_fn = lambda: fused(h)                                                   # noqa: E731
    for fn in (unfused_fn, fused_fn):
        for _ in range(3):
            fn()
    torch.cuda.synchronize()
    t_unfused = _timed(unfused_fn, steps, stream)
    t_fused = _timed(fused_fn, steps, stream)
    t_gq = _timed(lambda: kernels.quant_rows_fp8_gelu(h.view(LQ, FFN)), steps, stream)
    tunable.enable(False)
    out["ffn_gelu_down_8960x1536"] = {"ms": round(t_fused, 4), "unfused_ms": round(t_unfused, 4),
                                      "gelu_act_quant_call_ms": round(t_gq, 4), "gemm_table": table}
    # the MXFP8 mode (per-32 E8M0 scales) at the projection shape: its GEMM pads the rows to 128
    from lingbot_world_v2_realtime_amd.layers.linear import MXFP8Linear
    lin = torch.nn.Linear(DIM, DIM).to(torch.bfloat16).to(dev)
    f = MXFP8Linear(lin)
    x = torch.randn(1, LQ, DIM, device=dev).to(torch.bfloat16)
    for _ in range(3):
        f(x)
    torch.cuda.synchronize()
    ms = _timed(lambda: f(x), steps, torch.cuda.current_stream(dev))
    tf = 2.0 * LQ * DIM * DIM / (ms * 1e-3) / 1e12
    out["mx_proj_1536x1536"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                                "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4)}
    return out


def dropin_call(dev, lk=27144, calls=20):
    """The drop-in `attention()` call the reference ships (LINGBOT_ATTN=sage: sageattn over the bf16 window,
    lingbot/layers/attention.py:31-36): q [1,6032,12,128] against the reference's default 27144-key window, the
    whole window re-quantised on every call as sageattn does. HIP events around `calls` calls; the reference
    measured 2.090 ms for the same call on its GPU (experiments/bench_attn/results/h1.json)."""
    import torch
    from lingbot_world_v2_realtime_amd import sage_attention
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(1, n, H, D, device=dev, generator=g).to(torch.bfloat16) for n in (LQ, lk, lk))
    for _ in range(3):
        sage_attention(q, k, v)
    torch.cuda.synchronize()
    ms = _timed(lambda: sage_attention(q, k, v), calls, torch.cuda.current_stream(dev))
    ops = attention_ops(LQ, lk)
    return {"lq": LQ, "lk": lk, "ms": round(ms, 4), "TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
            "includes": "whole-window K/V re-quant + Q quant + attention, per call",
            "reference_ms_same_call": 2.090}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU emulation baseline")
    ap.add_argument("--cpu-heads", type=int, default=3)
    ap.add_argument("--no-sweep", action="store_true", help="skip the graph-captured per-chunk sweep")
    ap.add_argument("--table", action="store_true",
                    help="add the per-config GPU / CPU table (cfg 1, cfg 2 attention; cfg 4 layer; cfg 5 composed)")
    ap.add_argument("--only", choices=["attn", "requant", "prologue", "cross", "copy"],
                    help="profiling run: after the set-up, launch only this part --steps times and print its "
                         "mean time (copy: a 2 GiB device-to-device copy, the byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the attention path shards by head with no communication inside the "
              "op, and this build runs on one MI355X; use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from lingbot_world_v2_realtime_amd import _lib, kernels
    from lingbot_world_v2_realtime_amd.layers.kv_quant import QuantKVRing

    build = _lib.sources_sha16()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.only:
        return profile_only(args, dev)
    q, k, v, mem = synthetic_inputs(LQ, CHUNK, h=H, seed=0, mem_chunks=MEM, chunk_len=CHUNK)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    ring = QuantKVRing(1, 1, H, CHUNK, slots=MEM + 1, device=dev)
    for mk, mv in mem:
        ring.write(0, mk.to(dev), mv.to(dev))
        ring.commit()
    del mem

    def step():
        ring.write(0, k, v)
        return ring.attend(q, 0)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / args.steps * 1e3
    # the timed steps: the same step captured once as a HIP graph and replayed (all of its launches each time),
    # the form a DiT forward runs it in; the eager loop above pays a launch gap between each of its six kernels
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step()
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) / args.steps * 1e3
    del graph
    ops = attention_ops(LQ, LK, H, D)
    tops = ops / (ms_step * 1e-3) / 1e12

    # attention kernel alone, HIP events on the stream it is launched on
    slots, lens, _ = ring.attended()
    q8, qs, bias = kernels.quant_q(q, "NHD", ring.cache, 0, slots)
    o = torch.empty_like(q)
    stream = torch.cuda.current_stream(dev)
    for _ in range(5):
        kernels.attn_fwd(q8, qs, bias, 1, LQ, H, ring.cache, 0, slots, lens, o)
    attn_ms = _timed(lambda: kernels.attn_fwd(q8, qs, bias, 1, LQ, H, ring.cache, 0, slots, lens, o),
                     max(args.steps, 20), stream)
    attn_tops = ops / (attn_ms * 1e-3) / 1e12

    # K/V re-quant, 30 layers in one call (cfg 4)
    kl = torch.randn(LAYERS, 1, CHUNK, H, D, device=dev).to(torch.bfloat16)
    vl = torch.randn(LAYERS, 1, CHUNK, H, D, device=dev).to(torch.bfloat16)
    rq = QuantKVRing(LAYERS, 1, H, CHUNK, slots=MEM + 1, device=dev)
    for _ in range(3):
        rq.write_layers(kl, vl)
    rq_ms = _timed(lambda: rq.write_layers(kl, vl), 10, stream)
    rq_bytes = LAYERS * requant_bytes(CHUNK, H, D)
    rq_moved = LAYERS * requant_moved_bytes(CHUNK, H, D)
    rq_gbps = rq_bytes / (rq_ms * 1e-3) / 1e9
    del kl, vl, rq

    res = {
        "metric": "attn TOPS & % INT8 MFMA peak @6032q×24128kv d128; K/V requant GB/s",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "eager_ms_per_step": round(eager_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 QK / fp8-e4m3 PV (+ bf6 V residual), fp32 accumulate",
        "data": "synthetic, seeded (Q,V~N(0,1); K~N(0,1)+N(0,3) channel offset; memory ~N(0,1.5))",
        "config": {"workload": "chunk attending to memory: Q [1,6032,12,128] x 24128 keys (current chunk + "
                               "3 cached int8-K/fp8-V chunks); step = current-chunk K/V quant + Q quant + "
                               "attention kernel, replayed as one HIP graph", "lq": LQ, "lk": LK, "heads": H,
                   "head_dim": D},
        "roofline": {"bound": "mfma", "achieved": round(attn_tops, 2), "peak": MFMA_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(attn_tops / MFMA_PEAK_TOPS, 4),
                     "traffic": None,
                     "kernel": "lbw_attn_fwd = attn_fwd_kernel + attn_merge_kernel", "kernel_ms": round(attn_ms, 4),
                     "ops_per_launch": ops, "build_sha16": build},
        "requant": {"layers": LAYERS, "ms": round(rq_ms, 4), "algorithmic_bytes": rq_bytes,
                    "GB/s": round(rq_gbps, 1), "frac_hbm": round(rq_gbps / HBM_PEAK_GBPS, 4),
                    "bytes_moved": rq_moved, "GB/s_moved": round(rq_moved / (rq_ms * 1e-3) / 1e9, 1),
                    "frac_hbm_moved": round(rq_moved / (rq_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                    "note": "frac_hbm: algorithmic bytes (K, V read once; one V plane written); "
                            "frac_hbm_moved: the bytes the passes move (K read twice, two V planes, partials)"},
    }
    # traffic and counters come from rocprofv3 runs committed in profiles/; they count only when those runs
    # measured this very build (same source fingerprint), and the line says which build they are from
    traffic, traffic_build = traffic_from_profiles(build)
    res["roofline"]["traffic"] = traffic
    res["roofline"]["traffic_source"] = {"file": "profiles/attn_fwd_cfg3_traffic.json", "build_sha16": traffic_build,
                                         "matches_this_build": traffic_build == build}
    ctr = counters_from_profiles(build)
    if ctr is not None:   # issued MFMA work from the counters, over this run's HIP-event time
        issued = ctr["issued_ops"]
        res["roofline"]["counters"] = {
            "issued_ops_per_launch": issued, "issued_over_algorithmic": round(issued / ops, 4),
            "issued_TOPS": round(issued / (attn_ms * 1e-3) / 1e12, 1),
            "issued_frac": round(issued / (attn_ms * 1e-3) / 1e12 / MFMA_PEAK_TOPS, 4),
            "mfma_busy": round(ctr["mfma_busy"], 4), "profiled_kernel_ms": ctr.get("kernel_ms"),
            "source": "profiles/attn_fwd_cfg3_counters.json", "build_sha16": ctr["sources_sha16"]}
    res["prologue"] = prologue_call(dev, ring)
    res["cross_attention"] = cross_attention_call(dev)
    res["fp8_linear"] = fp8_linear_calls(dev)
    res["dropin_call"] = dropin_call(dev)
    res["chunk_sweep"] = None if args.no_sweep else chunk_sweep(dev)
    res["chunk_sweep_fused"] = None if args.no_sweep else chunk_sweep_fused(dev)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args.cpu_heads)
    else:
        res["cpu_baseline"] = None
    if args.table:
        res["config_table"] = config_table(dev, attn_ms, rq_ms,
                                           res["chunk_sweep"]["s_per_chunk"] if res["chunk_sweep"] else None,
                                           res["cpu_baseline"], args.cpu_heads)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
