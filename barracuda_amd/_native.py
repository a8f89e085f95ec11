"""ctypes binding of libbarracuda_hip.so (include/barracuda_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libbarracuda_hip.so"
HEADER = PKG.parent / "include" / "barracuda_hip.h"

BCH_OK = 0
BCH_E_INVALID = 1
BCH_E_SHAPE = 2
BCH_E_NO_DEVICE = 3
BCH_E_OOM = 4
BCH_E_MODULE = 5
BCH_E_LAUNCH = 6
BCH_E_DEVICE = 7
BCH_E_UNSUPPORTED = 8
BCH_E_DEVICE_LOST = 9
BCH_ACT_NONE = 0
BCH_ACT_RELU = 1
BCH_ACT_GELU = 2
BCH_EW_ADD, BCH_EW_SUB, BCH_EW_MUL, BCH_EW_NEG, BCH_EW_FMA, BCH_EW_SCALE, BCH_EW_RELU, BCH_EW_GELU = range(8)

_vp = C.c_void_p
_i = C.c_int
_ll = C.c_longlong
_sz = C.c_size_t
_f = C.c_float



class AttnLayout(C.Structure):
    """bch_attn_layout: element (b, h, i, d) at b*batch + h*head + i*row + d."""
    _fields_ = [("batch_stride", C.c_longlong), ("head_stride", C.c_longlong), ("row_stride", C.c_longlong)]


# name -> (restype, argtypes)
SIGNATURES = {
    "bch_device_count": (_i, [C.POINTER(_i)]),
    "bch_ctx_create": (_i, [_i, C.c_char_p, C.POINTER(_vp)]),
    "bch_ctx_destroy": (None, [_vp]),
    "bch_ctx_is_lost": (_i, [_vp, C.POINTER(_i)]),
    "bch_ctx_stream": (_i, [_vp, C.POINTER(_vp)]),
    "bch_ctx_reserve": (_i, [_vp, _sz]),
    "bch_ctx_workspace_bytes": (_i, [_vp, C.POINTER(_sz)]),
    "bch_last_error": (C.c_char_p, [_vp]),
    "bch_status_string": (C.c_char_p, [_i]),
    "bch_alloc": (_i, [_vp, _sz, C.POINTER(_vp)]),
    "bch_free": (_i, [_vp, _vp]),
    "bch_upload": (_i, [_vp, _vp, _vp, _sz]),
    "bch_download": (_i, [_vp, _vp, _vp, _sz]),
    "bch_memset": (_i, [_vp, _vp, _i, _sz]),
    "bch_sync": (_i, [_vp]),
    "bch_copy": (_i, [_vp, _vp, _vp, _sz]),
    "bch_sgemm": (_i, [_vp, _i, _i, _i, _vp, _i, _vp, _i, _vp, _i]),
    "bch_sgemm_noalloc": (_i, [_vp, _i, _i, _i, _vp, _i, _vp, _i, _vp, _i]),
    "bch_sgemm_ex": (_i, [_vp, _i, _i, _i, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i]),
    "bch_sgemm_strided_batched": (_i, [_vp, _i, _i, _i, _i, _vp, _ll, _vp, _ll, _vp, _ll]),
    "bch_dgemm": (_i, [_vp, _i, _i, _i, _i, _i, _i, C.c_double, _vp, _i, _ll, _vp, _i, _ll, C.c_double, _vp,
                       _i, _ll]),
    "bch_softmax_rows": (_i, [_vp, _ll, _ll, _vp, _vp]),
    "bch_softmax_rows_f64": (_i, [_vp, _ll, _ll, _vp, _vp]),
    "bch_elementwise": (_i, [_vp, _i, _ll, _vp, _vp, _vp, _f, _vp]),
    "bch_layer_norm": (_i, [_vp, _ll, _ll, _f, _vp, _vp]),
    "bch_layer_norm_kernel_name": (C.c_char_p, [_ll, _ll, _vp, _vp]),
    "bch_softmax_rows_f64_kernel_name": (C.c_char_p, [_ll, _ll, _vp, _vp]),
    "bch_softmax_axis": (_i, [_vp, _ll, _ll, _ll, _vp, _vp]),
    "bch_head_split": (_i, [_vp, _i, _i, _i, _i, _vp, _vp]),
    "bch_head_concat": (_i, [_vp, _i, _i, _i, _i, _vp, _vp]),
    "bch_sdpa_fwd": (_i, [_vp, _i, _i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _vp]),
    "bch_sdpa_fwd_ex": (_i, [_vp, _i, _i, _i, _i, _i, _i, _f, _i, _vp, AttnLayout, _vp, AttnLayout, _vp,
                             AttnLayout, _vp, AttnLayout]),
    "bch_launch_code_object": (_i, [_vp, _vp, _sz, C.c_char_p, C.POINTER(C.c_uint),
                                    C.POINTER(C.c_uint), C.POINTER(_vp), _sz, _sz]),
    "bch_event_create": (_i, [_vp, C.POINTER(_vp)]),
    "bch_event_record": (_i, [_vp, _vp]),
    "bch_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(_f)]),
    "bch_event_destroy": (None, [_vp]),
    "bch_sgemm_kernel_name": (C.c_char_p, [_i, _i, _i]),
    "bch_fill_uniform": (_i, [_vp, _vp, _sz, C.POINTER(C.c_ulonglong), C.c_double, C.c_double]),
    "bch_fill_normal": (_i, [_vp, _vp, _sz, C.POINTER(C.c_ulonglong), C.c_double, C.c_double]),
}

_lib = None


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bch_[a-z0-9_]+)\s*\(", text)))


def load() -> C.CDLL:
    """Load the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("BARRACUDA_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise RuntimeError(
            f"libbarracuda_hip.so not found at {path}: build it with "
            "`python -m barracuda_amd.build` (there is no CPU fallback)")
    lib = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error(ctx=None) -> str:
    msg = load().bch_last_error(ctx)
    return msg.decode() if msg else ""
