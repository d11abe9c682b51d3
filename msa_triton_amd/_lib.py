"""Loader for the C-ABI library ``libmsa_mi355x.so`` (hand-written gfx950 HIP kernels).

The library exports plain ``extern "C"`` entry points (declared in
``include/msa_mi355x.h``) that take raw device pointers, int64 sizes, scalars and
a ``hipStream_t``. This module binds them with ctypes. PyTorch is only used for
device memory and the current stream; there is no fallback path: if the library
is missing or fails to load, every operator raises.

torch is imported first on purpose: its bundled HIP runtime has the same soname
(``libamdhip64.so.7``) the library links against, so the dynamic loader binds
the library to the runtime torch already initialised (one runtime per process).
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_NAME = "libmsa_mi355x.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)
_lock = threading.Lock()
_lib = None

_vp, _i64, _f64, _i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double, ctypes.c_int32

# name -> (restype, argtypes); kept in sync with include/msa_mi355x.h
SIGNATURES = {
    "msa_topk": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "msa_k2q_counter_elems": (_i64, [_i64, _vp, _i64]),
    "msa_k2q_build": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                             _vp, _vp, _vp, _vp, _vp]),
    "msa_k2q_build_noalloc": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _vp, _vp, _vp, _vp]),
    "msa_split_block_indices": (_i32, [_vp, _i64, _i64, _i32, _vp, _vp]),
    "msa_score_fwd_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "msa_score_fwd": (_i32, [_vp, _vp, _i32, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f64,
                             _vp, _vp, _vp, _vp]),
    "msa_index_score_topk": (_i32, [_vp, _vp, _i32, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f64, _i64, _i64,
                                    _vp, _vp, _vp, _vp, _vp]),
    "msa_score_bwd": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                             _i64, _i64, _f64, _vp, _vp, _vp, _vp]),
    "msa_score_bwd_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "msa_attn_fwd_workspace_bytes": (_i64, [_i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "msa_attn_fwd": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i64, _f64, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp]),
    "msa_attn_bwd_workspace_bytes": (_i64, [_i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "msa_attn_bwd": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _f64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "msa_indexer_kl_workspace_bytes": (_i64, [_i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "msa_indexer_kl": (_i32, [_vp, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _f64, _f64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "msa_set_chunk_budgets": (_i32, [_i64, _i64, _i64]),
    "msa_set_item_order": (_i32, [_i32]),
    "msa_profile_begin": (_i32, []),
    "msa_profile_end": (_i64, [_vp, _vp, _i64]),
}

# Kernel kinds of msa_profile_end, in order.
PROFILE_KINDS = ("fwd_plan", "attn_fwd_partial_kernel", "attn_fwd_combine", "bwd_plan", "kv_bwd_center",
                 "kv_bwd_stats_kernel", "kv_bwd_stats_combine", "kv_bwd_main_kernel", "kv_bwd_accumulate",
                 "kv_bwd_dq_combine")

STATUS_TEXT = {1: "invalid argument", 2: "unsupported configuration", 3: "HIP launch failure"}

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def library_path() -> str:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Return the loaded native library, raising if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"{_LIB_NAME} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "(the MI355X kernels have no fallback path)"
                )
            handle = ctypes.CDLL(_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(status: int, name: str) -> None:
    if status != 0:
        raise RuntimeError(f"{name} failed: {STATUS_TEXT.get(status, status)}")


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(tensor: torch.Tensor, what: str) -> None:
    """The operators run only as HIP kernels on a ROCm device; CPU tensors raise."""
    if tensor.device.type != "cuda":
        raise RuntimeError(
            f"{what}: MI355X HIP kernels require ROCm device tensors (got {tensor.device}); "
            "there is no CPU execution path"
        )


class chunk_budgets:
    """Context manager over ``msa_set_chunk_budgets`` (a testing hook): runs the body with
    the given per-chunk record budgets in bytes for the KV-major attention forward,
    backward and indexer KL (None keeps a pass's default), then restores the defaults."""

    def __init__(self, fwd: int | None = None, bwd: int | None = None, kl: int | None = None):
        self.values = tuple(0 if x is None else int(x) for x in (fwd, bwd, kl))

    def __enter__(self):
        check(lib().msa_set_chunk_budgets(*self.values), "msa_set_chunk_budgets")
        return self

    def __exit__(self, *exc):
        lib().msa_set_chunk_budgets(0, 0, 0)
        return False


class row_order:
    """Context manager over ``msa_set_item_order`` (a testing hook): inside the body the
    KV-major passes launch their work items in row order instead of largest first."""

    def __enter__(self):
        check(lib().msa_set_item_order(0), "msa_set_item_order")
        return self

    def __exit__(self, *exc):
        lib().msa_set_item_order(1)
        return False


class kernel_timer:
    """Context manager over the library's profiling hook (``msa_profile_begin`` /
    ``msa_profile_end``): every kernel the attention entry points launch inside the body
    is timed with HIP events on its stream. After exit, ``ms`` and ``launches`` map each
    kernel kind of PROFILE_KINDS to its summed duration and launch count."""

    def __enter__(self):
        check(lib().msa_profile_begin(), "msa_profile_begin")
        self.ms, self.launches = {}, {}
        return self

    def __exit__(self, *exc):
        n = len(PROFILE_KINDS)
        ms = (ctypes.c_double * n)()
        launches = (ctypes.c_int64 * n)()
        got = lib().msa_profile_end(ms, launches, n)
        if got < 0:
            raise RuntimeError("msa_profile_end failed to read its events")
        self.ms = {name: ms[i] for i, name in enumerate(PROFILE_KINDS)}
        self.launches = {name: launches[i] for i, name in enumerate(PROFILE_KINDS)}
        return False
