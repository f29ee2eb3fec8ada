"""ctypes binding of libfmoe.so (the C ABI declared in include/fmoe.h).

The library links ``libamdhip64.so.7`` by soname.  torch-ROCm ships its own
copy of that runtime; importing torch first makes the loader bind libfmoe to
the runtime torch already uses, so device pointers and streams from torch
are valid in both.  ``hip_runtimes_loaded()`` lists the mapped copies so a
test can assert there is exactly one.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before libfmoe, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libfmoe.so"

# fmoe_status
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_SHAPE = 2
ERR_DTYPE = 3
ERR_IDS_RANGE = 4
ERR_NO_DEVICE = 5
ERR_HIP = 6
ERR_WORKSPACE = 7

# fmoe_dtype
F32 = 0
BF16 = 1
F8E4M3FN = 2
F8E4M3FN_A8 = 3  # block / sub-layer: e4m3 weights, prefill GEMMs on e4m3 activations
F8E4M3FN_A8X2 = 4  # the same with each activation as two e4m3 terms (hi + lo)

# fmoe_gemm_path
PATH_AUTO = 0
PATH_GENERIC = 1
PATH_TILED = 2
PATH_STREAM = 3
PATH_TILED_LARGE = 4


# FMOE_NOALLOC_SCRATCH_BYTES: the allocation-free block's fixed scratch size
NOALLOC_SCRATCH_BYTES = 64 << 20

# fmoe_timer
TIMERS = ("router", "permute", "gate_up", "down", "combine", "mul_mat_id", "norm", "qkv", "attention", "out_proj",
          "quant")


class FmoeError(RuntimeError):
    """A HIP-level failure reported by libfmoe (status FMOE_ERR_HIP)."""


class NoDeviceError(RuntimeError):
    """No usable gfx950 device (status FMOE_ERR_NO_DEVICE)."""


_EXC = {
    ERR_INVALID_ARGUMENT: ValueError,
    ERR_SHAPE: ValueError,
    ERR_DTYPE: TypeError,
    ERR_IDS_RANGE: IndexError,
    ERR_NO_DEVICE: NoDeviceError,
    ERR_HIP: FmoeError,
    ERR_WORKSPACE: ValueError,
}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "fmoe_last_error": (ctypes.c_char_p, []),
    "fmoe_abi_version": (_c_int, []),
    "fmoe_device_check": (_c_int, [ctypes.POINTER(_c_int), ctypes.c_char_p, _sz]),
    "fmoe_set_gemm_path": (_c_int, [_c_int]),
    "fmoe_get_gemm_path": (_c_int, []),
    "fmoe_last_gemm_path": (_c_int, []),
    "fmoe_quantize_rows_e4m3": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
    "fmoe_timing_enable": (_c_int, [_c_int]),
    "fmoe_timing_read": (_c_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_c_i64), _c_int]),
    "fmoe_swiglu": (_c_int, [_vp, _vp, _vp, _c_i64, _c_int, _vp]),
    "fmoe_router": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _vp, _vp, _vp]),
    "fmoe_permute_workspace_bytes": (_sz, [_c_i64, _c_i64, _c_i64]),
    "fmoe_permute": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _sz, _vp]),
    "fmoe_workspace_error_count": (_c_int, [_vp, _vp, ctypes.POINTER(_c_i64)]),
    "fmoe_packed_weight_bytes": (_sz, [_c_i64, _c_i64, _c_i64, _c_int]),
    "fmoe_pack_expert_weights": (_c_int, [_vp, _c_int, _vp, _c_i64, _c_i64, _c_i64, _c_int, _vp, _vp, _vp]),
    "fmoe_mul_mat_id_workspace_bytes": (_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "fmoe_mul_mat_id": (
        _c_int,
        [_vp, _vp, _c_int, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _vp, _sz, _vp],
    ),
    "fmoe_moe_ffn_block_workspace_bytes": (_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "fmoe_moe_ffn_block": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _vp, _sz, _vp],
    ),
    "fmoe_moe_ffn_block_noalloc": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _vp],
    ),
    "fmoe_rms_norm": (_c_int, [_vp, _vp, ctypes.c_float, _vp, _c_i64, _c_i64, _c_int, _vp]),
    "fmoe_moe_ffn_sublayer_workspace_bytes": (_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "fmoe_moe_ffn_sublayer": (
        _c_int,
        [_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _vp, _sz, _vp],
    ),
    "fmoe_moe_ffn_block_routing": (
        _c_int,
        [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
         ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp)],
    ),
    # decode attention half
    "fmoe_kvcache_gather": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
                 _vp, _vp],
    ),
    "fmoe_kvcache_scatter_decode": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_i64, _vp],
    ),
    "fmoe_kvcache_scatter_prefill": (
        _c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64,
                 _vp, _vp],
    ),
    "fmoe_pack_linear_weight": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _vp, _vp, _vp]),
    "fmoe_attention_block_decode_workspace_bytes": (_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "fmoe_attention_block_decode": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_i64, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _c_int,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, ctypes.c_float, _c_int, _vp, _vp, _vp, _vp, _sz,
         _vp],
    ),
    "fmoe_attention_decode_paged_workspace_bytes": (_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "fmoe_attention_sublayer_decode_paged_workspace_bytes": (
        _sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "fmoe_attention_sublayer_decode_paged": (
        _c_int,
        [_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp,
         _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _c_int,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, ctypes.c_float, _c_int, _vp, _vp, _vp, _vp, _sz,
         _vp],
    ),
    "fmoe_attention_decode_paged": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp,
         _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp, _vp, _c_int,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, ctypes.c_float, _c_int, _vp, _vp, _vp, _vp, _sz,
         _vp],
    ),
}

_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """Load libfmoe.so once.  Raises ImportError if it has not been built:
    there is no fallback implementation."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing; build it with __graft_entry__.build() "
                    "(python frank-models_amd/build.py)"
                )
            handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | ctypes.RTLD_LOCAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def last_error() -> str:
    return lib().fmoe_last_error().decode(errors="replace")


def check(status: int, what: str = "") -> None:
    if status != OK:
        exc = _EXC.get(status, FmoeError)
        msg = last_error()
        raise exc(f"{what}: {msg}" if what else msg)


def call(name: str, *args):
    """Call a status-returning entry point and raise on failure."""
    check(getattr(lib(), name)(*args), name)


def hip_runtimes_loaded():
    """Paths of every libamdhip64 mapped into this process."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in parts[5]:
                paths.add(os.path.realpath(parts[5]))
    return sorted(paths)


def timing_enable(on: bool = True) -> None:
    check(lib().fmoe_timing_enable(int(bool(on))), "fmoe_timing_enable")


def timing_read():
    """{kernel family: (total ms, timed regions)} since the last read (waits
    for the recorded HIP events).  A family can be timed in more than one
    region per call, so per-call times are totals divided by the calls."""
    n = len(TIMERS)
    ms = (ctypes.c_double * n)()
    cnt = (_c_i64 * n)()
    check(lib().fmoe_timing_read(ms, cnt, n), "fmoe_timing_read")
    return {name: (ms[i], cnt[i]) for i, name in enumerate(TIMERS)}
