"""C-ABI of liblbw_attn.so without a GPU: the library loads, exports every function include/lbw_attn.h declares
with the argument count the ctypes binding uses, and rejects bad arguments with the documented status codes
before touching the device."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from lingbot_world_v2_realtime_amd import _lib

HEADER = os.path.join(os.path.dirname(__file__), "..", "include", "lbw_attn.h")

OK, E_NULL, E_SHAPE, E_ALIGN, E_DEVICE, E_LAUNCH, E_SEGMENTS, E_SCRATCH = range(8)
FAKE = 1 << 20          # a 16-byte aligned non-null address; never dereferenced on the paths tested here


def declared_functions():
    """{name: number of parameters} of every function prototype in the header."""
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?\w+\s*\*?\s*(lbw_\w+)\s*\(([^)]*)\)\s*;", src, flags=re.M):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("liblbw_attn.so is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declarations_are_bound_and_exported(lib):
    decl = declared_functions()
    assert len(decl) == 18
    assert set(decl) == set(_lib.SIGNATURES)
    for name, n in decl.items():
        assert len(_lib.SIGNATURES[name][1]) == n, name
        assert hasattr(lib, name)
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line and "lbw_" in line}
    assert set(decl) <= exported


def test_status_strings_and_version(lib):
    names = [lib.lbw_status_string(s).decode() for s in range(8)]
    assert names[0] == "ok" and len(set(names)) == 8 and "unknown status" not in names
    assert lib.lbw_status_string(99).decode() == "unknown status"
    assert lib.lbw_version() == 100


def test_noalloc_scratch_size(lib):
    # the attention workspace of 8 XCDs x 32 workgroups: 2 partial slots of 256 rows x (128 channels + m, l)
    assert lib.lbw_attn_noalloc_scratch_bytes() == 8 * 32 * 2 * 256 * 130 * 4 == 68_157_440


def test_requant_workspace_formula(lib):
    for layers, bh, n in ((1, 1, 1), (30, 24, 1508), (2, 3, 64), (1, 5, 65), (30, 12, 6032), (1, 1, 262400)):
        nb = -(-n // 64)
        g = layers * bh
        # the K column sums of each 32-token half-block (V is quantised without a workspace)
        assert lib.lbw_kv_requant_workspace_bytes(layers, bh, n) == g * 2 * nb * 128 * 4
    assert lib.lbw_kv_requant_workspace_bytes(0, 1, 1) == 0


def requant(lib, **kw):
    a = dict(k=FAKE, v=FAKE, dtype=0, layers=1, batch=1, len=100, heads=2, ks=(0, 0, 256, 128),
             vs=(0, 0, 256, 128), k8=FAKE, k_scale=FAKE, km=FAKE, v8=FAKE, v8lo=None, v_scale=FAKE, slots=4, cap=128,
             slot=0, ws=FAKE)
    a.update(kw)
    return lib.lbw_kv_requant(a["k"], a["v"], a["dtype"], a["layers"], a["batch"], a["len"], a["heads"], *a["ks"], *a["vs"],
                              a["k8"], a["k_scale"], a["km"], a["v8"], a["v8lo"], a["v_scale"], a["slots"],
                              a["cap"], a["slot"], a["ws"], None)


def test_requant_argument_checks(lib):
    assert requant(lib, k=None) == E_NULL
    assert requant(lib, ws=None) == E_NULL
    assert requant(lib, len=0) == E_SHAPE
    assert requant(lib, len=129) == E_SHAPE            # more tokens than the slot holds
    assert requant(lib, cap=100) == E_SHAPE            # capacity not a multiple of 64
    assert requant(lib, slot=4) == E_SHAPE
    assert requant(lib, batch=300, heads=300) == E_SHAPE
    assert requant(lib, ks=(0, 0, 256, 129)) == E_ALIGN
    assert requant(lib, k8=FAKE + 8) == E_ALIGN
    assert requant(lib, v8lo=FAKE + 4) == E_ALIGN
    assert requant(lib, v_scale=FAKE + 2) == E_ALIGN  # the V scale table is stored as dwords
    assert requant(lib, dtype=2) == E_SHAPE            # bf16 (0) or fp16 (1) only


def quant_q(lib, **kw):
    a = dict(q=FAKE, dtype=0, batch=1, lq=100, heads=2, st=(0, 256, 128), q8=FAKE, qs=FAKE, km=FAKE, slots=4,
             n_seg=0, seg=None, bias=FAKE)
    a.update(kw)
    return lib.lbw_quant_q(a["q"], a["dtype"], a["batch"], a["lq"], a["heads"], *a["st"], a["q8"], a["qs"], a["km"],
                           a["slots"], a["n_seg"], a["seg"], a["bias"], None)


def test_quant_q_argument_checks(lib):
    seg = (ctypes.c_int32 * 2)(0, 5)
    assert quant_q(lib, q=None) == E_NULL
    assert quant_q(lib, lq=0) == E_SHAPE
    assert quant_q(lib, n_seg=9) == E_SEGMENTS
    assert quant_q(lib, st=(0, 256, 12)) == E_ALIGN
    assert quant_q(lib, n_seg=2, seg=None) == E_NULL
    assert quant_q(lib, n_seg=2, seg=seg) == E_SEGMENTS   # slot 5 of a 4-slot cache
    assert quant_q(lib, n_seg=2, seg=seg, km=FAKE + 4) == E_ALIGN   # the K means are read as float4
    assert quant_q(lib, dtype=-1) == E_SHAPE


ROPE_ROWS = 1024


def norm_rope_q(lib, **kw):
    a = dict(q=FAKE, batch=1, lq=100, heads=2, st=(0, 256), w=FAKE, eps=1e-6, rope=FAKE, rows=ROPE_ROWS,
             grid=(5, 4), f0=0, q8=FAKE, qs=FAKE, km=FAKE, slots=4, n_seg=0, seg=None, bias=FAKE, q_out=None,
             os=(0, 256, 128))
    a.update(kw)
    return lib.lbw_norm_rope_quant_q(a["q"], a["batch"], a["lq"], a["heads"], *a["st"], a["w"], a["eps"], a["rope"],
                                     a["rows"], *a["grid"], a["f0"], a["q8"], a["qs"], a["km"], a["slots"],
                                     a["n_seg"], a["seg"], a["bias"], a["q_out"], *a["os"], None)


def norm_rope_kv(lib, **kw):
    a = dict(k=FAKE, v=FAKE, batch=1, len=100, heads=2, ks=(0, 256), vs=(0, 256, 128), w=FAKE, eps=1e-6,
             rope=FAKE, rows=ROPE_ROWS, grid=(5, 4), f0=0, k_out=FAKE, os=(0, 256, 128), k8=FAKE, k_scale=FAKE,
             km=FAKE, v8=FAKE, v8lo=None, v_scale=FAKE, slots=4, cap=128, slot=0, ws=FAKE)
    a.update(kw)
    return lib.lbw_norm_rope_kv_requant(a["k"], a["v"], a["batch"], a["len"], a["heads"], *a["ks"], *a["vs"], a["w"],
                                        a["eps"], a["rope"], a["rows"], *a["grid"], a["f0"], a["k_out"], *a["os"],
                                        a["k8"], a["k_scale"], a["km"], a["v8"], a["v8lo"], a["v_scale"],
                                        a["slots"], a["cap"], a["slot"], a["ws"], None)


def test_norm_rope_argument_checks(lib):
    for call in (norm_rope_q, norm_rope_kv):
        assert call(lib, w=None) == E_NULL
        assert call(lib, rope=None) == E_NULL
        assert call(lib, heads=17) == E_SHAPE                   # one wave per head, at most 16
        assert call(lib, grid=(0, 4)) == E_SHAPE
        assert call(lib, f0=-1) == E_SHAPE
        assert call(lib, f0=ROPE_ROWS - 4) == E_SHAPE           # 100 tokens of 20-token frames need 5 frame rows
        assert call(lib, grid=(ROPE_ROWS + 1, 1)) == E_SHAPE    # the height index would run past the table
        assert call(lib, eps=float("nan")) == E_SHAPE
        assert call(lib, rope=FAKE + 8) == E_ALIGN
        assert call(lib, w=FAKE + 2) == E_ALIGN
    assert norm_rope_q(lib, st=(0, 252)) == E_ALIGN
    assert norm_rope_q(lib, q8=None) == E_NULL
    assert norm_rope_q(lib, n_seg=9) == E_SEGMENTS
    assert norm_rope_q(lib, n_seg=2, seg=(ctypes.c_int32 * 2)(0, 4)) == E_SEGMENTS
    assert norm_rope_q(lib, q_out=FAKE, os=(0, 256, 12)) == E_ALIGN
    assert norm_rope_kv(lib, k_out=None) == E_NULL
    assert norm_rope_kv(lib, ws=None) == E_NULL
    assert norm_rope_kv(lib, len=129) == E_SHAPE                # more tokens than the slot holds
    assert norm_rope_kv(lib, slot=4) == E_SHAPE
    assert norm_rope_kv(lib, vs=(0, 256, 12)) == E_ALIGN
    assert norm_rope_kv(lib, k8=FAKE + 8) == E_ALIGN
    assert norm_rope_kv(lib, v_scale=FAKE + 1) == E_ALIGN


def cross(lib, **kw):
    a = dict(q=FAKE, batch=1, lq=100, heads=2, qs=(0, 256, 128), kp=FAKE, vt=FAKE, lk=512, lens=None, out=FAKE,
             os=(0, 256, 128), sm=0.088)
    a.update(kw)
    return lib.lbw_cross_attn_fwd(a["q"], a["batch"], a["lq"], a["heads"], *a["qs"], a["kp"], a["vt"], a["lk"],
                                  a["lens"], a["out"], *a["os"], a["sm"], None)


def test_cross_attention_argument_checks(lib):
    assert cross(lib, q=None) == E_NULL
    assert cross(lib, vt=None) == E_NULL
    assert cross(lib, lk=0) == E_SHAPE
    assert cross(lib, batch=65) == E_SHAPE                     # per-batch key counts travel in the arguments
    assert cross(lib, sm=0.0) == E_SHAPE
    assert cross(lib, sm=float("inf")) == E_SHAPE
    assert cross(lib, lens=(ctypes.c_int32 * 1)(0)) == E_SHAPE  # each count 1 .. lk
    assert cross(lib, lens=(ctypes.c_int32 * 1)(513)) == E_SHAPE
    assert cross(lib, qs=(0, 256, 12)) == E_ALIGN
    assert cross(lib, out=FAKE + 4) == E_ALIGN
    prep = lambda **kw: lib.lbw_cross_prepare(kw.get("k", FAKE), FAKE, 1, kw.get("lk", 512), 2,  # noqa: E731
                                              0, 256, kw.get("ksh", 128), 0, 256, 128, FAKE, FAKE, None)
    assert prep(k=None) == E_NULL
    assert prep(lk=0) == E_SHAPE
    assert prep(ksh=130) == E_ALIGN


def test_quant_rows_fp8_argument_checks(lib):
    q = lambda **kw: lib.lbw_quant_rows_fp8(kw.get("x", FAKE), 0, kw.get("rows", 10), kw.get("cols", 256),  # noqa: E731
                                            kw.get("s", 256), kw.get("x8", FAKE), FAKE, None)
    assert q(x=None) == E_NULL
    assert q(rows=0) == E_SHAPE
    assert q(cols=100) == E_SHAPE          # multiples of 16, as the reference converts
    assert q(s=128) == E_SHAPE             # rows would overlap
    assert q(s=260) == E_ALIGN
    assert q(x=FAKE + 8) == E_ALIGN
    if hip_device_count() == 0:
        assert q() == E_DEVICE
    gq = lambda **kw: lib.lbw_quant_rows_fp8_gelu(kw.get("x", FAKE), kw.get("rows", 10), kw.get("cols", 256),  # noqa: E731
                                                  kw.get("s", 256), kw.get("x8", FAKE), kw.get("sc", FAKE), None)
    assert gq(sc=None) == E_NULL
    assert gq(cols=100) == E_SHAPE
    assert gq(s=128) == E_SHAPE
    assert gq(x8=FAKE + 4) == E_ALIGN
    if hip_device_count() == 0:
        assert gq() == E_DEVICE
    mx = lambda **kw: lib.lbw_quant_mx_fp8(kw.get("x", FAKE), 0, kw.get("rows", 10), kw.get("pad", 128),  # noqa: E731
                                           kw.get("cols", 256), kw.get("s", 256), kw.get("x8", FAKE), FAKE, None)
    assert mx(x=None) == E_NULL
    assert mx(cols=48) == E_SHAPE          # whole 32-value groups
    assert mx(pad=5) == E_SHAPE            # the padded row count holds every row
    assert mx(s=200) == E_SHAPE
    assert mx(x8=FAKE + 8) == E_ALIGN
    if hip_device_count() == 0:
        assert mx() == E_DEVICE


def attn(lib, logits=None, **kw):
    seg = (ctypes.c_int32 * 8)(0, 1, 2, 3, 0, 0, 0, 0)
    ln = (ctypes.c_int32 * 8)(128, 128, 128, 100, 0, 0, 0, 0)
    a = dict(q8=FAKE, qs=FAKE, bias=FAKE, batch=1, lq=100, heads=2, k8=FAKE, ks=FAKE, v8=FAKE, v8lo=None,
             vs=FAKE, slots=4, cap=128, n_seg=4, seg=seg, ln=ln, first=None, out=FAKE, os=(0, 256, 128), sm=0.088,
             ws=FAKE)
    a.update(kw)
    args = (a["q8"], a["qs"], a["bias"], a["batch"], a["lq"], a["heads"], a["k8"], a["ks"], a["v8"], a["v8lo"],
            a["vs"], a["slots"], a["cap"], a["n_seg"], a["seg"], a["ln"], a["first"], a["out"], *a["os"], a["sm"])
    if logits is not None:   # the checking build: the same arguments plus the logits output
        return lib.lbw_qk_logits_i32(*args, logits, a["ws"], None)
    return lib.lbw_attn_fwd(*args, a["ws"], None)


def test_attn_argument_checks(lib):
    assert attn(lib, q8=None) == E_NULL
    assert attn(lib, ws=None) == E_NULL
    assert attn(lib, bias=None) == E_NULL                 # several chunks need the q . mean bias
    assert attn(lib, cap=96) == E_SHAPE
    assert attn(lib, sm=0.0) == E_SHAPE
    assert attn(lib, sm=float("nan")) == E_SHAPE
    assert attn(lib, n_seg=0) == E_SEGMENTS
    assert attn(lib, n_seg=9) == E_SEGMENTS
    assert attn(lib, ln=(ctypes.c_int32 * 8)(128, 129, 1, 1, 0, 0, 0, 0)) == E_SEGMENTS
    assert attn(lib, ln=(ctypes.c_int32 * 8)(128, 0, 1, 1, 0, 0, 0, 0)) == E_SEGMENTS
    assert attn(lib, seg=(ctypes.c_int32 * 8)(0, 1, 2, 4, 0, 0, 0, 0)) == E_SEGMENTS
    assert attn(lib, os=(0, 256, 130)) == E_ALIGN
    assert attn(lib, out=FAKE + 2) == E_ALIGN
    assert attn(lib, v8=FAKE + 8) == E_ALIGN
    assert attn(lib, vs=FAKE + 2) == E_ALIGN              # the V scale table is read as dwords
    # first tokens: a chunk read from token `first` must end inside its slot
    first = lambda *f: (ctypes.c_int32 * 8)(*f, *[0] * (8 - len(f)))  # noqa: E731
    assert attn(lib, first=first(0, 0, 0, 29)) == E_SEGMENTS          # 29 + 100 > 128
    assert attn(lib, first=first(0, -1, 0, 0)) == E_SEGMENTS
    assert attn(lib, first=first(0, 0, 1, 0)) == E_SEGMENTS           # 1 + 128 > 128
    # the checking build takes the same checks, and its logits output
    assert attn(lib, logits=FAKE, q8=None) == E_NULL
    assert attn(lib, logits=0) == E_NULL                                # a null logits pointer
    assert attn(lib, logits=FAKE + 2) == E_ALIGN
    assert attn(lib, logits=FAKE, first=first(0, 0, 0, 29)) == E_SEGMENTS


def hip_device_count():
    """Devices the HIP runtime itself reports (not torch's view: a CPU-only torch on a GPU host sees none).
    Any doubt counts as a device, so the caller skips."""
    if os.path.exists("/dev/kfd"):
        return 1
    # in a fresh interpreter: once torch is imported, its own HIP runtime clashes with a second one loaded here
    probe = ("import ctypes, os\n"
             "hip = ctypes.CDLL(os.path.join(os.environ.get('ROCM_PATH', '/opt/rocm'), 'lib', 'libamdhip64.so'))\n"
             "n = ctypes.c_int(0)\n"
             "rc = hip.hipGetDeviceCount(ctypes.byref(n))\n"
             "print(n.value if rc == 0 else 0)\n")
    res = subprocess.run([sys.executable, "-c", probe], capture_output=True, text=True)
    try:
        return int(res.stdout.strip()) if res.returncode == 0 else 1
    except ValueError:
        return 1


def test_valid_call_without_gfx950_is_refused(lib):
    """With arguments that pass every check, a process that sees no gfx950 device gets LBW_E_DEVICE and no
    launch. Runs only where the HIP runtime reports no device: on a GPU host these calls would launch kernels on
    fake pointers."""
    if hip_device_count() != 0:
        pytest.skip("the HIP runtime reports a device")
    assert requant(lib) == E_DEVICE
    assert quant_q(lib) == E_DEVICE
    assert attn(lib) == E_DEVICE
    assert norm_rope_q(lib) == E_DEVICE
    assert norm_rope_kv(lib) == E_DEVICE
    assert cross(lib) == E_DEVICE
    assert lib.lbw_cross_prepare(FAKE, FAKE, 1, 512, 2, 0, 256, 128, 0, 256, 128, FAKE, FAKE, None) == E_DEVICE
    seg = (ctypes.c_int32 * 1)(0)
    ln = (ctypes.c_int32 * 1)(100)
    first = (ctypes.c_int32 * 1)(28)
    assert lib.lbw_attn_fwd_noalloc(FAKE, FAKE, None, 1, 100, 2, FAKE, FAKE, FAKE, None, FAKE, 1, 128, 1, seg, ln,
                                    first, FAKE, 0, 256, 128, 0.088, None) == E_DEVICE
    assert attn(lib, first=(ctypes.c_int32 * 8)(0, 0, 0, 28, 0, 0, 0, 0)) == E_DEVICE
    assert attn(lib, logits=FAKE) == E_DEVICE


def test_loader_fails_loudly_without_library(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(ImportError):
        _lib.load(str(tmp_path / "missing.so"))
