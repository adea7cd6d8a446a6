"""The committed golden fixtures (tests/golden/golden.npz, written by tests/golden/make_golden.py): the oracle
must still reproduce them (CPU), and the HIP path must match them -- bit for bit for the quantised tensors,
scales and int32 logits, and within the oracle-distance bound for the attention outputs (GPU)."""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import emu

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
import make_golden  # noqa: E402

DEV = "cuda"


@pytest.fixture(scope="module")
def gold():
    return make_golden.load()


def _mem(gold):
    return [(gold["mem0_k"], gold["mem0_v"]), (gold["mem1_k"], gold["mem1_v"])]


def test_oracle_reproduces_fixtures(gold):
    r = emu.requant(gold["k"], gold["v"])
    for name in ("k8", "k_scale", "km", "v8", "v8lo", "v_scale"):
        assert np.array_equal(r[name].numpy(), gold[name]), name
    q8, qs = emu.quant_q(gold["q"])
    assert np.array_equal(q8.numpy(), gold["q8"]) and np.array_equal(qs.numpy(), gold["q_scale"])
    assert np.array_equal(emu.qk_logits(q8, r["k8"])[:, :, :100].numpy(), gold["logits"])
    gx = int(gold["gx"])
    a1 = emu.attention(gold["q"], [r], schedule_gx=gx).numpy()
    chunks = [emu.requant(mk, mv) for mk, mv in _mem(gold)] + [r]
    ring = emu.attention(gold["q"], chunks, schedule_gx=gx).numpy()
    # fp32 GEMMs on the host may differ in the last bits between CPUs
    assert np.abs(a1 - gold["attn1"]).max() < 1e-5
    assert np.abs(ring - gold["ring"]).max() < 1e-5


def _attention_bound(out, ref, sd):
    """The HIP output sits within a small fraction of the scheme's distance from fp32 SDPA of the oracle."""
    e_emu, e_scheme = (out - ref).abs(), (ref - sd).abs()
    print(f"vs-oracle max {e_emu.max():.3e} mean {e_emu.mean():.3e}; oracle vs-sdpa mean {e_scheme.mean():.3e}")
    assert e_emu.mean() <= 0.1 * e_scheme.mean() + 2e-3 * sd.abs().mean()
    assert e_emu.max() <= e_scheme.max() + 2e-3


@pytest.mark.gpu
def test_hip_matches_fixtures(gold):
    from lingbot_world_v2_realtime_amd import _lib, kernels
    from lingbot_world_v2_realtime_amd.layers.kv_quant import QuantKVRing
    h = gold["k"].shape[2]
    ring = kernels.RingCache(1, 1, h, 128, 1, DEV)
    kernels.kv_requant(gold["k"].to(DEV), gold["v"].to(DEV), ring, 0)
    q8, qs, _ = kernels.quant_q(gold["q"].to(DEV))
    raw, _ = kernels.qk_logits(q8, qs, None, 1, 70, h, ring, 0, [0], [100])
    logits = raw - kernels.S_MAGIC   # the attention kernel's accumulator words, less their start value
    torch.cuda.synchronize()
    assert np.array_equal(ring.km[0, 0].cpu().numpy(), gold["km"])
    assert np.array_equal(ring.v_scale[0, 0, :, :2].cpu().numpy(), gold["v_scale"])
    assert np.array_equal(ring.k_scale[0, 0, :, :2].cpu().numpy(), gold["k_scale"])
    assert np.array_equal(ring.k8[0, 0].cpu().numpy(), gold["k8"])
    assert np.array_equal(ring.v8[0, 0].cpu().numpy(), gold["v8"])
    assert np.array_equal(ring.v8lo[0, 0].cpu().numpy(), gold["v8lo"])
    assert np.array_equal(q8.cpu().numpy(), gold["q8"]) and np.array_equal(qs.cpu().numpy(), gold["q_scale"])
    assert np.array_equal(logits[:, :, :100].cpu().numpy(), gold["logits"])

    same_schedule = _lib.load().lbw_attn_workgroups_per_xcd() == int(gold["gx"])
    gx = _lib.load().lbw_attn_workgroups_per_xcd()
    q = gold["q"]
    out = kernels.attn_fwd(q8, qs, None, 1, 70, h, ring, 0, [0], [100], torch.empty(1, 70, h, 128,
                           dtype=torch.bfloat16, device=DEV)).float().cpu()[0]
    ref = torch.from_numpy(gold["attn1"]) if same_schedule else \
        emu.attention(q, [emu.requant(gold["k"], gold["v"])], schedule_gx=gx)
    _attention_bound(out, ref, emu.sdpa_fp32(q, gold["k"], gold["v"]))

    mem = _mem(gold)
    qr = QuantKVRing(1, 1, h, 100, slots=4, device=DEV)
    for mk, mv in mem:
        qr.write(0, mk.to(DEV), mv.to(DEV))
        qr.commit()
    qr.write(0, gold["k"].to(DEV), gold["v"].to(DEV))
    out = qr.attend(q.to(DEV), 0).float().cpu()[0]
    chunks = [emu.requant(mk, mv) for mk, mv in mem] + [emu.requant(gold["k"], gold["v"])]
    ref = torch.from_numpy(gold["ring"]) if same_schedule else emu.attention(q, chunks, schedule_gx=gx)
    kk = torch.cat([m[0] for m in mem] + [gold["k"]], 1)
    vv = torch.cat([m[1] for m in mem] + [gold["v"]], 1)
    _attention_bound(out, ref, emu.sdpa_fp32(q, kk, vv))
