"""ctypes binding of libflexatt.so, the C ABI declared in include/flexatt.h.

This is the only bridge between the Python API and the HIP kernels.  There is
no fallback: if the library is missing or fails to load, every entry point
raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libflexatt.so")

F32, F16, BF16 = 0, 1, 2

# Entry points declared in include/flexatt.h.
EXPORTS = (
    "flexatt_fwd",
    "flexatt_fwd_decode_workspace",
    "flexatt_fwd_decode",
    "flexatt_fwd_decode_noalloc",
    "flexatt_bwd_delta",
    "flexatt_bwd_dq",
    "flexatt_bwd_dq_delta",
    "flexatt_bwd_dkdv",
    "flexatt_bwd",
    "flexatt_bwd_workspace",
    "flexatt_bwd_workspace_limited",
    "flexatt_bwd_prefers_staging",
    "flexatt_bwd_ws",
    "flexatt_bwd_dkdv_ds",
    "flexatt_bwd_dq_ds",
    "flexatt_status_string",
    "flexatt_abi_version",
)
ABI_VERSION = 8
# Fixed scratch of flexatt_fwd_decode_noalloc (FLEXATT_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 16 << 20
# Work-queue counters at the end of the staged-dS workspace (FLEXATT_BWD_QUEUE_BYTES).
BWD_QUEUE_BYTES = 256


class Tensor(ctypes.Structure):
    """``flexatt_tensor``: device pointer + element strides of [B, H, S, D]."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_s", ctypes.c_int64),
        ("stride_d", ctypes.c_int64),
    ]


class Problem(ctypes.Structure):
    """``flexatt_problem``: sizes, dtype and mask primitives."""

    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("sliding_window", ctypes.c_int32),
        ("soft_cap", ctypes.c_float),
        ("alibi_slopes", ctypes.c_void_p),
        ("doc_bounds", ctypes.c_void_p),
        ("col_bounds", ctypes.c_void_p),
        ("block_map", ctypes.c_void_p),
        ("block_heads", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_lib = None


def load() -> ctypes.CDLL:
    """Load libflexatt.so once and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libflexatt.so not found at {LIB_PATH}: build it with "
            "`python npu-flex-att_amd/build_lib.py` or `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    import torch  # noqa: F401  (binds the process to torch's HIP runtime first)

    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER
    T = P(Tensor)
    pr = P(Problem)
    fp = ctypes.c_void_p
    st = ctypes.c_void_p
    sig = {
        "flexatt_fwd": [pr, T, T, T, T, fp, st],
        "flexatt_fwd_decode": [pr, T, T, T, T, fp, fp, ctypes.c_size_t, st],
        "flexatt_fwd_decode_noalloc": [pr, T, T, T, T, fp, st],
        "flexatt_bwd_delta": [pr, T, T, fp, st],
        "flexatt_bwd_dq": [pr, T, T, T, T, fp, fp, T, st],
        "flexatt_bwd_dq_delta": [pr, T, T, T, T, T, fp, fp, T, st],
        "flexatt_bwd_dkdv": [pr, T, T, T, T, fp, fp, T, T, st],
        "flexatt_bwd": [pr, T, T, T, T, T, fp, fp, T, T, T, st],
        "flexatt_bwd_ws": [pr, T, T, T, T, T, fp, fp, T, T, T, fp, ctypes.c_size_t, st],
        "flexatt_bwd_dkdv_ds": [pr, T, T, T, T, fp, fp, T, T, fp, ctypes.c_size_t, st],
        "flexatt_bwd_dq_ds": [pr, T, fp, ctypes.c_size_t, T, st],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    for name in ("flexatt_fwd_decode_workspace", "flexatt_bwd_workspace"):
        getattr(lib, name).argtypes = [pr]
        getattr(lib, name).restype = ctypes.c_size_t
    lib.flexatt_bwd_workspace_limited.argtypes = [pr, ctypes.c_size_t]
    lib.flexatt_bwd_workspace_limited.restype = ctypes.c_size_t
    lib.flexatt_bwd_prefers_staging.argtypes = [pr]
    lib.flexatt_bwd_prefers_staging.restype = ctypes.c_int
    lib.flexatt_status_string.argtypes = [ctypes.c_int]
    lib.flexatt_status_string.restype = ctypes.c_char_p
    lib.flexatt_abi_version.argtypes = []
    lib.flexatt_abi_version.restype = ctypes.c_int
    if lib.flexatt_abi_version() != ABI_VERSION:
        raise RuntimeError("libflexatt.so ABI version mismatch; rebuild the library")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    """Raise RuntimeError for a non-zero flexatt status."""
    if status != 0:
        msg = load().flexatt_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def tensor(t) -> Tensor:
    """Describe a 4-D torch tensor for the C ABI (no copy)."""
    sb, sh, ss, sd = t.stride()
    return Tensor(t.data_ptr(), sb, sh, ss, sd)
