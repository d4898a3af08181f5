"""ctypes view of libgdn_hip.so's C ABI (include/gdn_hip.h, include/gdn_hip_diag.h).

This is the binding a Python caller of the reference's C entry points would
write; the tests use it to call the boundary directly with raw device
pointers, and to check that every declared symbol is exported.
"""
from __future__ import annotations

import ctypes as ct
import re
from pathlib import Path

from . import LIB_PATH

INCLUDE = Path(__file__).resolve().parents[2] / "include"
HEADERS = sorted(INCLUDE.glob("*.h"))

hipError_t = ct.c_int
hipStream_t = ct.c_void_p
vp, fp, i32p = ct.c_void_p, ct.c_void_p, ct.c_void_p
c_int, c_size_t, c_int64, c_float = ct.c_int, ct.c_size_t, ct.c_int64, ct.c_float

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
HIP_ERROR_LAUNCH_TIMEOUT = 702
DTYPE_BF16, DTYPE_FP16, DTYPE_FP32 = 0, 1, 2

_PROTOS = {
    "deltanet_prefill_workspace_size": (c_size_t, [c_int] * 6),
    "deltanet_tcop_prefill_workspace_size": (c_size_t, [c_int] * 6),
    "deltanet_chunk_prefill": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp] + [c_int] * 7 +
                               [vp, c_size_t, hipStream_t, c_int]),
    "deltanet_tcop_chunk_prefill": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp] + [c_int] * 7 +
                                    [vp, c_size_t, hipStream_t, c_int]),
    "deltanet_prefill_live_workspace_size": (c_size_t, [c_int] * 6),
    "deltanet_chunk_prefill_norm": (hipError_t, [vp, vp, vp, fp, fp, vp, vp, c_float, vp, fp, fp] +
                                    [c_int] * 7 + [vp, c_size_t, hipStream_t]),
    "deltanet_chunk_prefill_norm_fused": (hipError_t, [vp, vp, vp, fp, fp, vp, vp, c_float, vp,
                                                       fp, fp] + [c_int] * 7 +
                                          [vp, c_size_t, hipStream_t]),
    "deltanet_chunk_prefill_noalloc": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp] +
                                       [c_int] * 7 + [hipStream_t]),
    "deltanet_prefill_noalloc_status": (hipError_t, [hipStream_t]),
    "deltanet_prefill_varlen_workspace_size": (c_size_t, [c_int] * 6),
    "deltanet_prefill_varlen_live_workspace_size": (c_size_t, [c_int] * 6),
    "deltanet_prefill_status": (hipError_t, [vp, c_size_t, hipStream_t]),
    "deltanet_chunk_prefill_spin": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp] + [c_int] * 4 +
                                    [vp, c_size_t, hipStream_t, ct.c_uint]),
    "deltanet_chunk_prefill_cols": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp, vp] + [c_int] * 4 +
                                    [vp, c_size_t, hipStream_t, c_int, ct.c_uint]),
    "deltanet_varlen_chunk_map": (c_int, [vp, c_int, c_int, vp, vp, vp, vp]),
    "deltanet_varlen_chunks_before": (c_int, [vp, c_int, c_int, c_int, c_int]),
    "deltanet_prefill_twolevel_workspace_size": (c_size_t, [vp, c_int, c_int, c_int, c_int]),
    "deltanet_chunk_prefill_twolevel": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp, vp] +
                                        [c_int] * 5 + [vp, c_size_t, hipStream_t, vp, c_int]),
    "deltanet_varlen_locate_chunk": (c_int, [vp, c_int, c_int, c_int, c_int, vp]),
    "deltanet_chunk_prefill_varlen": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp, i32p] +
                                      [c_int] * 7 + [vp, c_size_t, hipStream_t, c_int]),
    "deltanet_recurrent_step": (hipError_t, [vp, vp, vp, fp, fp, vp, fp] + [c_int] * 6 +
                                [hipStream_t]),
    "deltanet_recurrent_step_l2norm": (hipError_t, [vp, vp, vp, fp, fp, vp, fp] + [c_int] * 6 +
                                       [hipStream_t]),
    "deltanet_prefill_kernel_count": (c_int, []),
    "deltanet_prefill_kernel_name": (ct.c_char_p, [c_int]),
    "deltanet_chunk_prefill_timed": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp] + [c_int] * 7 +
                                     [vp, c_size_t, hipStream_t, vp, c_int]),
    "deltanet_chunk_prefill_kernel": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp] + [c_int] * 7 +
                                      [vp, c_size_t, hipStream_t, c_int]),
    "deltanet_chunk_prefill_l2norm": (hipError_t, [vp, vp, vp, fp, fp, vp, fp, fp, i32p] +
                                      [c_int] * 5 + [vp, c_size_t, hipStream_t]),
    "deltanet_chunk_prefill_fused": (hipError_t, [vp, vp, vp, vp, vp, fp, vp, vp, fp] +
                                     [c_int] * 5 + [vp, c_size_t, hipStream_t]),
    "gdn_gated_rmsnorm_forward": (hipError_t, [vp, vp, vp, vp, c_int64, c_int, c_float, c_int,
                                               c_int, hipStream_t]),
    "gdn_causal_conv1d_fwd": (hipError_t, [vp, vp, vp, vp] + [c_int] * 4 + [c_int64] * 4 +
                              [c_int] * 3 + [hipStream_t]),
    "gdn_stream_probe": (hipError_t, [c_int, c_int, vp, vp, vp, c_size_t, c_int, hipStream_t]),
    "gdn_causal_conv1d_update": (hipError_t, [vp, vp, vp, vp, vp] + [c_int] * 5 + [c_int64] * 8 +
                                 [c_int] * 3 + [hipStream_t]),
}


def declared_symbols() -> list[str]:
    """Function names declared in include/*.h."""
    names = []
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:size_t|hipError_t|int|const char\s*\*)\s*(\w+)\s*\(",
                            text, flags=re.M)
    return names


_lib = None


def lib() -> ct.CDLL:
    global _lib
    if _lib is None:
        _lib = ct.CDLL(str(LIB_PATH))
        for name, (res, args) in _PROTOS.items():
            f = getattr(_lib, name)
            f.restype = res
            f.argtypes = args
    return _lib


def ptr(t) -> int | None:
    """Raw data pointer of a torch tensor (None for None)."""
    return None if t is None else t.data_ptr()
