"""ctypes binding of the C ABI in include/sa.h (libsa_hip.so, built in-tree next to this file).

The library is loaded once per process. Nothing here falls back to another implementation: when
the shared object is missing or fails to load, `load()` raises RuntimeError with the reason, and
the operator entry points in `kernels` refuse to run.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libsa_hip.so"
# SA_HIP_LIBRARY names another build of the same library (for example one compiled with other
# tile or group defaults); by default the in-tree build next to this file is loaded.
LIB_PATH = os.environ.get("SA_HIP_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

DTYPE_BF16 = 0
DTYPE_F32 = 1

# Kernel ids of sa_timing_read.
KERNEL_FORWARD = 0
KERNEL_BACKWARD = 1
KERNEL_SELECTION = 2
KERNEL_BACKWARD_DQ = 3
KERNEL_DECODE = 4

class ViewStrides(ctypes.Structure):
    """sa_view_strides: element strides of a (sequence, head, row) view."""

    _fields_ = [("seq", ctypes.c_int64), ("head", ctypes.c_int64), ("row", ctypes.c_int64)]


# Every function the header declares, with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_VS = ctypes.POINTER(ViewStrides)
SIGNATURES = {
    "sa_abi_version": (_I, []),
    "sa_status_string": (ctypes.c_char_p, [_I]),
    "sa_transposed_ld": (_I64, [_I64]),
    "sa_timing_enable": (_I, [_I]),
    "sa_timing_read": (_I, [_I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I64)]),
    "sa_forward_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I, _I]),
    "sa_forward": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64,
                        _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _I, _I, _I64, _P]),
    "sa_forward_strided": (_I, [_P, _VS, _P, _VS, _P, _VS, _P, _P, _VS, _P, _P, _P, _P, _P, _I64, _P, _I64,
                                _I64, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _I, _I, _I64, _P]),
    "sa_backward_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I, _I]),
    "sa_backward_strided": (_I, [_P, _VS, _P, _VS, _P, _VS, _P, _P, _VS, _P, _P, _P, _P, _VS, _P, _VS, _P, _VS,
                                 _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _I, _I, _P]),
    "sa_backward": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                         _I64, _I64, _I64, _I64, _F, _I, _I, _I, _I, _P]),
    "sa_decode_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "sa_decode": (_I, [_P, _P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _P]),
    "sa_decode_noalloc": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _P]),
}

# Bytes of the fixed device scratch of sa_decode_noalloc (SA_DECODE_SCRATCH_BYTES).
DECODE_SCRATCH_BYTES = 64 << 20

_lock = threading.Lock()
_lib = None
_error: str | None = None


def load() -> ctypes.CDLL:
    """The loaded library; RuntimeError when it cannot be loaded."""

    global _lib, _error
    with _lock:
        if _lib is not None:
            return _lib
        if _error is not None:
            raise RuntimeError(_error)
        if not os.path.exists(LIB_PATH):
            _error = (f"the HIP kernel library {LIB_PATH} is not built "
                      "(run __graft_entry__.build() or selective-attention-study_amd/csrc/build.sh)")
            raise RuntimeError(_error)
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as exc:  # missing ROCm runtime, wrong architecture, ...
            _error = f"cannot load {LIB_PATH}: {exc}"
            raise RuntimeError(_error) from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
    except RuntimeError:
        return False
    return True


def check(status: int) -> None:
    """Raise RuntimeError for a non-zero status from the C ABI."""

    if status != 0:
        lib = load()
        raise RuntimeError(f"selective attention HIP call failed ({status}): "
                           f"{lib.sa_status_string(status).decode()}")


def timing_enable(on: bool) -> None:
    """Discard recorded kernel timings and switch event recording on or off."""

    check(load().sa_timing_enable(1 if on else 0))


def timing_read(kernel: int) -> tuple[float, int]:
    """(summed milliseconds, launches) recorded for one kernel id since timing_enable."""

    total = ctypes.c_double(0.0)
    count = ctypes.c_int64(0)
    check(load().sa_timing_read(kernel, ctypes.byref(total), ctypes.byref(count)))
    return total.value, count.value
