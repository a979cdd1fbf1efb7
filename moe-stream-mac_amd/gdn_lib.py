"""ctypes binding to ``libgdn_mi355x.so`` (C ABI declared in ``include/gdn_mi355x.h``).

torch is imported before the library is opened so that the library binds to the HIP runtime torch already
loaded (both carry the soname ``libamdhip64.so.7``); device pointers and streams are then shared.
There is no fallback: a missing library is an error.
"""

from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = Path(__file__).resolve().parent / "libgdn_mi355x.so"
HEADER = Path(__file__).resolve().parent.parent / "include" / "gdn_mi355x.h"

GDN_OK, GDN_ERR_INVALID, GDN_ERR_UNSUPPORTED, GDN_ERR_WORKSPACE, GDN_ERR_LAUNCH = 0, -1, -2, -3, -4
F32, BF16, F16 = 0, 1, 2
GATE_DECAY, GATE_DECAY_VEC, GATE_LOG, GATE_LOG_VEC = 0, 1, 2, 3
FORM_AUTO, FORM_RECURRENT, FORM_CHUNK = 0, 1, 2
FORMS = {"auto": FORM_AUTO, "recurrent": FORM_RECURRENT, "chunk": FORM_CHUNK}

DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t
_SIGS = {
    "gdn_gates_fwd": ([_vp] * 6 + [_i64, _i, _i, _i, _i, _vp], _i),
    "gdn_gates_bwd_workspace_bytes": ([_i64, _i], _sz),
    "gdn_gates_bwd": ([_vp] * 12 + [_sz, _i64, _i, _i, _i, _i, _i, _vp], _i),
    "gdn_l2norm_fwd": ([_vp, _vp, _i64, _i, _f, _f, _i, _vp], _i),
    "gdn_l2norm_bwd": ([_vp, _vp, _vp, _i64, _i, _f, _f, _i, _i, _vp], _i),
    "gdn_conv_silu_fwd": ([_vp] * 5 + [_i] * 5 + [_vp], _i),
    "gdn_conv_silu_bwd_workspace_bytes": ([_i] * 4, _sz),
    "gdn_conv_silu_bwd": ([_vp] * 7 + [_sz] + [_i] * 6 + [_vp], _i),
    "gdn_conv_qkv_fwd": ([_vp] * 7 + [_i] * 7 + [_f, _f, _i, _vp], _i),
    "gdn_conv_qkv_bwd": ([_vp] * 9 + [_sz] + [_i] * 7 + [_f, _f, _i, _i, _vp], _i),
    "gdn_gated_rmsnorm_fwd": ([_vp] * 4 + [_i64, _i, _f, _i, _i, _vp], _i),
    "gdn_gated_rmsnorm_bwd_workspace_bytes": ([_i64, _i], _sz),
    "gdn_gated_rmsnorm_bwd": ([_vp] * 8 + [_sz, _i64, _i, _f, _i, _i, _i, _vp], _i),
    "gdn_version": ([], _i),
    "gdn_last_error": ([], ctypes.c_char_p),
    "gdn_num_snapshots": ([_i, _i], ctypes.c_int64),
    "gdn_select_form": ([_i] * 7, _i),
    "gdn_saved_bytes": ([_i] * 11, ctypes.c_size_t),
    "gdn_fwd_workspace_bytes": ([_i] * 12, ctypes.c_size_t),
    "gdn_fwd": ([_vp] * 10 + [_sz, _vp, _sz] + [_i] * 11 + [_vp], _i),
    "gdn_bwd_workspace_bytes": ([_i] * 11, ctypes.c_size_t),
    "gdn_decode_step": ([_vp] * 8 + [_i] * 8 + [_vp], _i),
    "gdn_fwd_noalloc": ([_vp] * 9 + [_i] * 10 + [_vp], _i),
    "gdn_bwd": ([_vp] * 8 + [ctypes.c_size_t] + [_vp] * 9 + [ctypes.c_size_t] + [_i] * 12 + [_vp], _i),
    "gdn_profile_enable": ([_i], _i),
    "gdn_profile_collect": ([_i, ctypes.c_char_p, _i, ctypes.POINTER(ctypes.c_double),
                             ctypes.POINTER(_i)], _i),
}

_lib = None


class GDNError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def load() -> ctypes.CDLL:
    """Open the library once; raises if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP engine first "
                "(python moe-stream-mac_amd/build.py or __graft_entry__.build())")
        lib = ctypes.CDLL(os.fspath(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def header_functions() -> list[str]:
    """Function names declared by include/gdn_mi355x.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(gdn_[a-z_0-9]+)\s*\(", text, re.M)))


def check(status: int) -> None:
    if status != GDN_OK:
        msg = load().gdn_last_error().decode(errors="replace")
        if status in (GDN_ERR_INVALID,):
            raise ValueError(msg)
        raise GDNError(status, msg)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def profile_enable(on: bool) -> None:
    load().gdn_profile_enable(1 if on else 0)


def profile_collect() -> dict[str, tuple[float, int]]:
    """{kernel: (total_ms, launches)} recorded since the last collect (waits for the events)."""
    n_max, name_len = 32, 64
    names = ctypes.create_string_buffer(n_max * name_len)
    ms = (ctypes.c_double * n_max)()
    counts = (ctypes.c_int * n_max)()
    n = load().gdn_profile_collect(n_max, names, name_len, ms, counts)
    if n < 0:
        check(n)
    out = {}
    for i in range(n):
        raw = names.raw[i * name_len:(i + 1) * name_len]
        out[raw.split(b"\0", 1)[0].decode()] = (ms[i], counts[i])
    return out


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
