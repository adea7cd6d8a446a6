"""ctypes binding of liblbw_attn.so (the C-ABI declared in include/lbw_attn.h)."""
import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liblbw_attn.so")

_i64, _i32, _f32, _p = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/lbw_attn.h
SIGNATURES = {
    "lbw_status_string": (ctypes.c_char_p, [_i32]),
    "lbw_version": (_i32, []),
    "lbw_kv_requant_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "lbw_kv_requant": (_i32, [_p, _p, _i32, _i64, _i64, _i64, _i64,
                              _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p]),
    "lbw_quant_q": (_i32, [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _i32, _p, _p, _p]),
    "lbw_norm_rope_quant_q": (_i32, [_p, _i64, _i64, _i64, _i64, _i64, _p, _f32, _p, _i64, _i64, _i64, _i64,
                                     _p, _p, _p, _i64, _i32, _p, _p, _p, _i64, _i64, _i64, _p]),
    "lbw_norm_rope_kv_requant": (_i32, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _f32,
                                        _p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                                        _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p]),
    "lbw_cross_prepare": (_i32, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p]),
    "lbw_cross_attn_fwd": (_i32, [_p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _i64, _i64, _i64,
                                  _f32, _p]),
    "lbw_quant_rows_fp8": (_i32, [_p, _i32, _i64, _i64, _i64, _p, _p, _p]),
    "lbw_quant_rows_fp8_gelu": (_i32, [_p, _i64, _i64, _i64, _p, _p, _p]),
    "lbw_quant_mx_fp8": (_i32, [_p, _i32, _i64, _i64, _i64, _i64, _p, _p, _p]),
    "lbw_attn_fwd": (_i32, [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p, _p, _p,
                            _p, _i64, _i64, _i64, _f32, _p, _p]),
    "lbw_attn_workspace_bytes": (_i64, []),
    "lbw_attn_fwd_noalloc": (_i32, [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p, _p, _p,
                                    _p, _i64, _i64, _i64, _f32, _p]),
    "lbw_attn_noalloc_scratch_bytes": (_i64, []),
    "lbw_attn_workgroups_per_xcd": (_i32, []),
    "lbw_qk_logits_i32": (_i32, [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p, _p, _p,
                                 _p, _i64, _i64, _i64, _f32, _p, _p, _p]),
}


def sources_sha16():
    """First 16 hex digits of a sha256 over what liblbw_attn.so is built from: the HIP sources and headers (csrc/,
    include/) and the compiler flags. A measurement stored with this fingerprint describes this build when the
    fingerprints match."""
    import hashlib
    from . import build
    here = os.path.dirname(os.path.abspath(__file__))
    files = [os.path.join(here, "csrc", f) for f in sorted(os.listdir(os.path.join(here, "csrc")))
             if f.endswith((".hip", ".h"))]
    files.append(os.path.join(os.path.dirname(here), "include", "lbw_attn.h"))
    h = hashlib.sha256(" ".join(build.HIPCC_FLAGS).encode())
    for f in files:
        with open(f, "rb") as fh:
            h.update(os.path.basename(f).encode() + b"\0" + fh.read())
    return h.hexdigest()[:16]


class LbwError(RuntimeError):
    pass


_LIB = None


def load(path=LIB_PATH):
    """Load liblbw_attn.so and bind its entry points; raises if the library was not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                          "or `python lingbot_world_v2_realtime_amd/build.py`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(status, what):
    if status != 0:
        msg = load().lbw_status_string(status).decode()
        raise LbwError(f"{what} failed: status {status} ({msg})")
