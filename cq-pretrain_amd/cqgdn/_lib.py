"""Bindings of libcqgdn.so (the C ABI declared in include/cqgdn.h).

* ``lib()``: the ctypes binding of every C-ABI symbol (workspace sizes, host helpers, the layer
  kernels, instrumentation);
* ``ops()``: ``torch.ops.cqgdn``, the PyTorch-ROCm operators of libcqgdn_torch.so
  (csrc/torch_ops.cpp, TORCH_LIBRARY(cqgdn)) through which the per-step calls go: the training
  forward and backward, the recurrent decode and the layer decode step.

Both libraries are loaded from this package directory (built in-tree by
``cq-pretrain_amd/build.py``).  There is no fallback: a missing library, or a
call that returns an error code, raises.
"""

from __future__ import annotations

import ctypes
import hashlib
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libcqgdn.so")
OPS_PATH = LIB_PATH.with_name("libcqgdn_torch.so")

OK, EINVAL, EUNSUPPORTED, EHIP = 0, 1, 2, 3
NORMALIZE, TRAINING, PRECISE, NO_OUTPUT, FP16 = 1, 2, 4, 8, 16
STATIC_WORKSPACE_BYTES = 64 << 20  # CQGDN_STATIC_WORKSPACE_BYTES
FWD_BUFFERS, BWD_BUFFERS = 9, 8
FWD_NAMES = ("rk", "gcum", "T", "W", "UT", "KgT", "hT", "vnT", "vscale")
BWD_NAMES = ("dvlT", "XT", "dh", "dVn", "knP", "WT", "sync", "dscale")

# every symbol include/cqgdn.h declares, with (restype, argtypes)
_P, _I, _I64, _U, _F, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "cqgdn_version": (ctypes.c_char_p, []),
    "cqgdn_last_error": (ctypes.c_char_p, []),
    "cqgdn_chunk_table": (_I64, [_P, _I, _P, _P]),
    "cqgdn_fwd_workspace_size": (_SZ, [_I64, _I, _I64]),
    "cqgdn_fwd_buffer_offsets": (_I, [_I64, _I, _I64, _P, _I]),
    "cqgdn_bwd_workspace_size": (_SZ, [_I64, _I, _I64]),
    "cqgdn_bwd_buffer_offsets": (_I, [_I64, _I, _I64, _P, _I]),
    "cqgdn_fwd": (_I, [_P, _P, _P, _P, _P, _I64, _I, _P, _I64, _P, _I, _F, _U, _P, _P, _P, _P, _SZ, _P]),
    "cqgdn_fwd_static": (_I, [_P, _P, _P, _P, _P, _I64, _I, _P, _I64, _P, _I, _F, _U, _P, _P, _P, _P]),
    "cqgdn_fwd_static_init": (_I, []),
    "cqgdn_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I, _P, _I64, _P, _I, _F, _U, _P, _SZ, _P, _SZ, _P, _P, _P, _P,
                       _P, _P]),
    "cqgdn_bwd_recompute": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I, _P, _I64, _P, _I, _F, _U, _P, _SZ, _P, _SZ, _P,
                                 _P, _P, _P, _P, _P]),
    "cqgdn_recurrent": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _F, _P]),
    "cqgdn_l2norm_fwd": (_I, [_P, _P, _P, _I64, _P]),
    "cqgdn_l2norm_bwd": (_I, [_P, _P, _P, _P, _I64, _P]),
    "cqgdn_chunk_local_cumsum": (_I, [_P, _P, _I64, _I, _P, _I64, _I, _P]),
    "cqgdn_conv1d_fwd": (_I, [_P, _P, _P, _I, _I64, _I, _I, _I, _P, _P]),
    "cqgdn_conv1d_bwd_workspace_size": (_SZ, [_I64, _I, _I]),
    "cqgdn_conv1d_bwd": (_I, [_P, _P, _P, _P, _I, _I64, _I, _I, _I, _P, _P, _P, _SZ, _P]),
    "cqgdn_gated_norm_fwd": (_I, [_P, _P, _I64, _I, _P, _I64, _P, _F, _P, _P, _P]),
    "cqgdn_gated_norm_bwd_workspace_size": (_SZ, [_I64, _I]),
    "cqgdn_gated_norm_bwd": (_I, [_P, _P, _P, _I64, _I64, _I, _P, _I64, _P, _P, _P, _P, _P, _I64, _P, _P, _SZ, _P]),
    "cqgdn_event_inputs_fwd_workspace_size": (_SZ, [_I, _I, _I]),
    "cqgdn_event_inputs_fwd": (_I, [_P, _I, _I, _P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "cqgdn_event_inputs_bwd_workspace_size": (_SZ, [_P, _I, _I]),
    "cqgdn_event_inputs_bwd": (_I, [_P, _I, _I, _P, _I64, _P, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                                    _P, _I64, _P, _I64, _P, _P, _P, _SZ, _P]),
    "cqgdn_layer_decode_workspace_size": (_SZ, [_I, _I]),
    "cqgdn_layer_decode_step": (_I, [_I, _I, _I, _I, _P, _I64, _P, _P, _P, _P, _P, _F, _F, _P, _P, _P, _SZ, _P]),
    "cqgdn_timer_arm": (_I, [ctypes.c_char_p, _I]),
    "cqgdn_timer_read": (_I, [_P, _I, _P]),
}
class EventPlan(ctypes.Structure):
    """struct cqgdn_event_plan of include/cqgdn.h."""

    _fields_ = [("n_content", ctypes.c_int32), ("n_queries", ctypes.c_int32), ("n_events", ctypes.c_int32),
                ("conv_kernel", ctypes.c_int32), ("content_order", _P), ("event_q", _P), ("event_write", _P),
                ("query_source", _P), ("query_history", _P), ("content_bounds", _P),
                ("n_content_docs", ctypes.c_int32), ("n_history_rows", ctypes.c_int32), ("q_ptr", _P),
                ("q_list", _P), ("write_event", _P), ("query_event", _P), ("history_ptr", _P),
                ("history_list", _P), ("history_rows", _P), ("n_fold_rows", ctypes.c_int32), ("fold_rows", _P),
                ("fold_ptr", _P), ("fold_list", _P)]


KERNELS = ("fwd_prep", "fwd_scan", "fwd_out", "bwd_local", "bwd_scan", "bwd_dkw", "recurrent")

_LIB = None
_OPS = None


class CqgdnError(RuntimeError):
    """A HIP runtime failure reported by libcqgdn."""


def lib():
    """Load libcqgdn.so once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python cq-pretrain_amd/build.py` "
                "(the hip GDN backend has no fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _LIB = handle
    return _LIB


def ops():
    """``torch.ops.cqgdn`` (fwd, bwd, recurrent, layer_decode_step), loaded once; raise if unbuilt."""
    global _OPS
    if _OPS is None:
        lib()  # the operator library links libcqgdn.so: load it (and check it exists) first
        if not OPS_PATH.exists():
            raise RuntimeError(f"{OPS_PATH} is missing: build it with `python cq-pretrain_amd/build.py` "
                               "(the hip GDN backend has no fallback)")
        import torch

        torch.ops.load_library(str(OPS_PATH))
        _OPS = torch.ops.cqgdn
    return _OPS


def check(rc: int, what: str) -> None:
    if rc == OK:
        return
    msg = f"{what}: {lib().cqgdn_last_error().decode()}"
    if rc == EINVAL:
        raise ValueError(msg)
    if rc == EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise CqgdnError(msg)


def version() -> str:
    return lib().cqgdn_version().decode()


def sha256() -> str:
    return hashlib.sha256(LIB_PATH.read_bytes()).hexdigest()


def fwd_offsets(T: int, H: int, n_chunks: int) -> dict:
    arr = (ctypes.c_size_t * FWD_BUFFERS)()
    check(lib().cqgdn_fwd_buffer_offsets(T, H, n_chunks, arr, FWD_BUFFERS), "cqgdn_fwd_buffer_offsets")
    return dict(zip(FWD_NAMES, arr))


def bwd_offsets(T: int, H: int, n_chunks: int) -> dict:
    arr = (ctypes.c_size_t * BWD_BUFFERS)()
    check(lib().cqgdn_bwd_buffer_offsets(T, H, n_chunks, arr, BWD_BUFFERS), "cqgdn_bwd_buffer_offsets")
    return dict(zip(BWD_NAMES, arr))


class KernelTimer:
    """Time every launch of one library kernel with hipEvents on its own stream.

    Usage: ``with KernelTimer("bwd_dkw", 64) as t: ...``; afterwards ``t.ms``
    holds the per-launch durations (the exit waits for the recorded events).
    """

    def __init__(self, kernel: str, max_launches: int):
        if kernel not in KERNELS:
            raise ValueError(f"unknown kernel {kernel!r}; one of {KERNELS}")
        self.kernel, self.max_launches, self.ms = kernel, max_launches, []

    def __enter__(self):
        rc = lib().cqgdn_timer_arm(self.kernel.encode(), self.max_launches)
        if rc != OK:
            raise CqgdnError(f"cqgdn_timer_arm({self.kernel}) failed with code {rc}")
        return self

    def __exit__(self, *exc):
        buf = (ctypes.c_float * self.max_launches)()
        n = ctypes.c_int(0)
        rc = lib().cqgdn_timer_read(buf, self.max_launches, ctypes.byref(n))
        if rc != OK and exc[0] is None:
            raise CqgdnError(f"cqgdn_timer_read({self.kernel}) failed with code {rc}")
        self.ms = list(buf[:n.value])
        return False
