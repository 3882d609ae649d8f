"""ctypes binding of ``libpallas_flash_amd.so`` (C ABI in include/pallas_flash_amd.h).

The structs below mirror the header field by field. There is no fallback: if
the library is missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
from typing import Iterator, Optional

import torch

_LIB_FILE = "libpallas_flash_amd.so"
_lib: Optional[ctypes.CDLL] = None

PF_OK = 0
PF_ERR_INVALID = -1
PF_ERR_UNSUPPORTED = -2
PF_ERR_WORKSPACE = -3
PF_ERR_LAUNCH = -4

PF_DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

c_i32 = ctypes.c_int32
c_f32 = ctypes.c_float
c_ptr = ctypes.c_void_p


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_ptr), ("k", c_ptr), ("v", c_ptr), ("o", c_ptr), ("lse", c_ptr),
        ("batch", c_i32), ("num_heads", c_i32), ("num_kv_heads", c_i32),
        ("seq_len_q", c_i32), ("seq_len_k", c_i32), ("head_dim", c_i32),
        ("kv_len", c_i32), ("causal", c_i32), ("sm_scale", c_f32), ("dtype", c_i32),
    ]


class FwdRopeArgs(ctypes.Structure):
    _fields_ = [
        ("base", FwdArgs),
        ("q_cos", c_ptr), ("q_sin", c_ptr), ("k_cos", c_ptr), ("k_sin", c_ptr),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_ptr), ("k", c_ptr), ("v", c_ptr), ("o", c_ptr), ("do_", c_ptr),
        ("lse", c_ptr), ("delta", c_ptr), ("dq", c_ptr), ("dk", c_ptr), ("dv", c_ptr),
        ("batch", c_i32), ("num_heads", c_i32), ("num_kv_heads", c_i32),
        ("seq_len_q", c_i32), ("seq_len_k", c_i32), ("head_dim", c_i32),
        ("kv_len", c_i32), ("causal", c_i32), ("sm_scale", c_f32), ("dtype", c_i32),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_ptr), ("k_cache", c_ptr), ("v_cache", c_ptr), ("o", c_ptr),
        ("batch", c_i32), ("num_heads", c_i32), ("num_kv_heads", c_i32),
        ("cache_size", c_i32), ("head_dim", c_i32), ("cache_len", c_i32),
        ("sm_scale", c_f32), ("dtype", c_i32),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
    ]


class PagedArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_ptr), ("k_pages", c_ptr), ("v_pages", c_ptr),
        ("block_tables", c_ptr), ("context_lens", c_ptr), ("o", c_ptr),
        ("batch", c_i32), ("num_heads", c_i32), ("num_kv_heads", c_i32),
        ("num_pages", c_i32), ("page_size", c_i32), ("head_dim", c_i32),
        ("pages_per_seq", c_i32), ("sm_scale", c_f32), ("dtype", c_i32),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
    ]


class RopeArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_ptr), ("out", c_ptr), ("cos", c_ptr), ("sin", c_ptr),
        ("batch", c_i32), ("heads", c_i32), ("seq_len", c_i32), ("head_dim", c_i32), ("rope_len", c_i32),
        ("inverse", c_i32), ("dtype", c_i32),
    ]


class KvWriteArgs(ctypes.Structure):
    _fields_ = [
        ("k", c_ptr), ("v", c_ptr), ("k_cache", c_ptr), ("v_cache", c_ptr),
        ("positions", c_ptr), ("positions_stride", c_i32),
        ("batch", c_i32), ("num_kv_heads", c_i32), ("seq_len", c_i32), ("cache_size", c_i32),
        ("head_dim", c_i32), ("ring", c_i32), ("dtype", c_i32),
    ]


class PagedWriteArgs(ctypes.Structure):
    _fields_ = [
        ("k", c_ptr), ("v", c_ptr), ("k_pages", c_ptr), ("v_pages", c_ptr),
        ("block_tables", c_ptr), ("positions", c_ptr), ("positions_stride", c_i32),
        ("batch", c_i32), ("num_kv_heads", c_i32), ("seq_len", c_i32), ("num_pages", c_i32),
        ("page_size", c_i32), ("head_dim", c_i32), ("pages_per_seq", c_i32), ("dtype", c_i32),
    ]


class DecodeStepArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_ptr), ("k_new", c_ptr), ("v_new", c_ptr), ("k_cache", c_ptr), ("v_cache", c_ptr),
        ("o", c_ptr), ("positions", c_ptr), ("positions_stride", c_i32),
        ("cos", c_ptr), ("sin", c_ptr), ("rope_len", c_i32),
        ("batch", c_i32), ("num_heads", c_i32), ("num_kv_heads", c_i32), ("cache_size", c_i32),
        ("head_dim", c_i32), ("ring", c_i32), ("sm_scale", c_f32), ("dtype", c_i32),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
    ]


class Tuning(ctypes.Structure):
    _fields_ = [("tail_dynamic_pct", c_i32), ("decode_stages", c_i32), ("decode_waves", c_i32)]


# (symbol, argtypes, restype) for every entry point the header declares.
SIGNATURES = {
    "pf_attn_fwd": ([ctypes.POINTER(FwdArgs), c_ptr], ctypes.c_int),
    "pf_attn_fwd_rope_workspace_size": ([ctypes.POINTER(FwdRopeArgs)], ctypes.c_size_t),
    "pf_attn_fwd_rope": ([ctypes.POINTER(FwdRopeArgs), c_ptr], ctypes.c_int),
    "pf_attn_bwd_delta": ([ctypes.POINTER(BwdArgs), c_ptr], ctypes.c_int),
    "pf_attn_bwd_dq": ([ctypes.POINTER(BwdArgs), c_ptr], ctypes.c_int),
    "pf_attn_bwd_dkv": ([ctypes.POINTER(BwdArgs), c_ptr], ctypes.c_int),
    "pf_attn_bwd": ([ctypes.POINTER(BwdArgs), c_ptr], ctypes.c_int),
    "pf_attn_decode_workspace_size": ([ctypes.POINTER(DecodeArgs)], ctypes.c_size_t),
    "pf_attn_decode": ([ctypes.POINTER(DecodeArgs), c_ptr], ctypes.c_int),
    "pf_paged_attn_workspace_size": ([ctypes.POINTER(PagedArgs)], ctypes.c_size_t),
    "pf_paged_attn": ([ctypes.POINTER(PagedArgs), c_ptr], ctypes.c_int),
    "pf_paged_attn_noalloc": ([ctypes.POINTER(PagedArgs), c_ptr], ctypes.c_int),
    "pf_rope": ([ctypes.POINTER(RopeArgs), c_ptr], ctypes.c_int),
    "pf_kv_cache_write": ([ctypes.POINTER(KvWriteArgs), c_ptr], ctypes.c_int),
    "pf_paged_cache_write": ([ctypes.POINTER(PagedWriteArgs), c_ptr], ctypes.c_int),
    "pf_attn_decode_step_workspace_size": ([ctypes.POINTER(DecodeStepArgs)], ctypes.c_size_t),
    "pf_attn_decode_step": ([ctypes.POINTER(DecodeStepArgs), c_ptr], ctypes.c_int),
    "pf_get_tuning": ([ctypes.POINTER(Tuning)], ctypes.c_int),
    "pf_set_tuning": ([ctypes.POINTER(Tuning)], ctypes.c_int),
    "pf_version": ([], ctypes.c_char_p),
}


def library_path() -> str:
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_FILE)


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built."""
    global _lib
    if _lib is None:
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"{_LIB_FILE} is not built (expected at {path}); run `make` in "
                "tpu-native-pallas-flashattention_amd/ or __graft_entry__.build()")
        handle = ctypes.CDLL(path)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Map a pf_status to a Python exception."""
    if status == PF_OK:
        return
    if status == PF_ERR_INVALID:
        raise ValueError(f"{what}: invalid arguments (rejected by the C ABI)")
    if status == PF_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: unsupported configuration (dtype or head_dim)")
    if status == PF_ERR_WORKSPACE:
        raise RuntimeError(f"{what}: workspace missing or too small")
    raise RuntimeError(f"{what}: HIP launch failed (status {status})")


def dtype_tag(t: torch.Tensor) -> int:
    try:
        return PF_DTYPE[t.dtype]
    except KeyError:
        raise NotImplementedError(
            f"dtype {t.dtype} is not supported (float32, bfloat16, float16)") from None


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(*tensors: torch.Tensor) -> None:
    """The kernels run on a ROCm device only; there is no CPU path."""
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                "pallas_flash (MI355X) runs its HIP kernels on ROCm device tensors only; "
                f"got a tensor on {t.device}")
        if t.device != dev:
            raise ValueError(f"all tensors must be on one device, got {dev} and {t.device}")


def get_tuning() -> dict:
    """The library's process-wide tuning (pf_get_tuning)."""
    t = Tuning()
    check(lib().pf_get_tuning(ctypes.byref(t)), "pf_get_tuning")
    return {name: getattr(t, name) for name, _ in Tuning._fields_}


@contextlib.contextmanager
def tuning(**overrides) -> Iterator[dict]:
    """Run a block with some tuning fields replaced (pf_set_tuning), restoring
    the previous values afterwards. Fields: tail_dynamic_pct (0..100),
    decode_stages (2..4), decode_waves (0 = one per resident slot, or the
    persistent decode grid size)."""
    old = get_tuning()
    new = dict(old)
    for name, value in overrides.items():
        if name not in new:
            raise TypeError(f"unknown tuning field {name!r}")
        new[name] = int(value)
    check(lib().pf_set_tuning(ctypes.byref(Tuning(**new))), "pf_set_tuning")
    try:
        yield new
    finally:
        check(lib().pf_set_tuning(ctypes.byref(Tuning(**old))), "pf_set_tuning")
