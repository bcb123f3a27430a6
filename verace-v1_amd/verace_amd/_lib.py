"""ctypes binding of libverace_sssd.so (the C ABI declared in include/verace_sssd.h).

The library is built in-tree by ``verace-v1_amd/build.py``.  torch is imported first
so that the HIP runtime torch ships with is the one the library binds to (both carry
the soname libamdhip64.so.7).  There is no fallback: if the library is missing or a
call fails, a RuntimeError names the cause.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libverace_sssd.so")

VMI_F32, VMI_BF16, VMI_F16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: VMI_F32, torch.bfloat16: VMI_BF16, torch.float16: VMI_F16}

EXPORTED = (
    "vmi_version",
    "vmi_status_string",
    "vmi_last_hip_error",
    "vmi_sssd_scan_workspace_bytes",
    "vmi_sssd_scan_fwd",
    "vmi_sssd_scan_fwd_noalloc",
    "vmi_sssd_scan_fused_workspace_bytes",
    "vmi_sssd_scan_fused",
    "vmi_sssd_step_inplace",
    "vmi_sssd_step_fused",
    "vmi_sssd_step_slots",
    "vmi_state_cache_create",
    "vmi_state_cache_destroy",
    "vmi_state_cache_new",
    "vmi_state_cache_fork",
    "vmi_state_cache_release",
    "vmi_state_cache_plan",
    "vmi_state_cache_slots",
    "vmi_state_cache_refs",
    "vmi_state_cache_step",
    "vmi_state_cache_attach_hologram",
    "vmi_state_cache_cham_workspace_bytes",
    "vmi_state_cache_cham_step",
    "vmi_cham_scan_workspace_bytes",
    "vmi_cham_scan_fwd",
    "vmi_cham_scan_fused",
    "vmi_sssd_scan_bwd_workspace_bytes",
    "vmi_sssd_scan_bwd",
    "vmi_cham_step_workspace_bytes",
    "vmi_cham_step_inplace",
    "vmi_cham_step_fused",
    "vmi_cham_ns_workspace_bytes",
    "vmi_cham_ns_retraction",
)

_lib = None
_load_error = None


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise RuntimeError(f"verace_amd: unsupported dtype {dt} (float32, bfloat16, float16)") from None


def _declare(lib):
    vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
    lib.vmi_version.argtypes = []
    lib.vmi_version.restype = i32
    lib.vmi_status_string.argtypes = [i32]
    lib.vmi_status_string.restype = ctypes.c_char_p
    lib.vmi_last_hip_error.argtypes = []
    lib.vmi_last_hip_error.restype = i32
    lib.vmi_sssd_scan_workspace_bytes.argtypes = [i64, i64, i64, i64, i32, ctypes.POINTER(sz)]
    lib.vmi_sssd_scan_workspace_bytes.restype = i32
    lib.vmi_sssd_scan_fwd.argtypes = [vp, vp, vp, vp, i32, i32, vp, vp, vp, i64, i64, i64, i64,
                                      vp, sz, vp]
    lib.vmi_sssd_scan_fwd.restype = i32
    lib.vmi_sssd_scan_fwd_noalloc.argtypes = [vp, vp, vp, vp, i32, i32, vp, vp, vp, i64, i64, i64,
                                              i64, vp]
    lib.vmi_sssd_scan_fwd_noalloc.restype = i32
    lib.vmi_sssd_scan_fused_workspace_bytes.argtypes = [i64, i64, i64, i64, i32, ctypes.POINTER(sz)]
    lib.vmi_sssd_scan_fused_workspace_bytes.restype = i32
    lib.vmi_sssd_scan_fused.argtypes = [vp, i64, i32, vp, vp, ctypes.c_float, vp, vp, vp, i64, i64,
                                        i64, i64, vp, sz, vp]
    lib.vmi_sssd_scan_fused.restype = i32
    lib.vmi_sssd_step_inplace.argtypes = [vp, vp, vp, vp, i32, i32, vp, vp, i64, i64, i64, vp]
    lib.vmi_sssd_step_fused.argtypes = [vp, i64, i32, vp, vp, ctypes.c_float, vp, vp, i64, i64, i64,
                                        vp]
    lib.vmi_sssd_step_fused.restype = i32
    lib.vmi_sssd_step_inplace.restype = i32
    lib.vmi_sssd_step_slots.argtypes = [vp, vp, vp, vp, i32, i32, vp, i64, vp, vp, vp, i64, i64,
                                        i64, vp]
    lib.vmi_sssd_step_slots.restype = i32
    pi64 = ctypes.POINTER(i64)
    pi32 = ctypes.POINTER(i32)
    lib.vmi_state_cache_create.argtypes = [i64, i64, i64, i64, vp, ctypes.POINTER(vp)]
    lib.vmi_state_cache_destroy.argtypes = [vp]
    lib.vmi_state_cache_new.argtypes = [vp, i64, pi64]
    lib.vmi_state_cache_fork.argtypes = [vp, i64, i64, pi64]
    lib.vmi_state_cache_release.argtypes = [vp, pi64, i64]
    lib.vmi_state_cache_plan.argtypes = [vp, i64, pi64, i64, pi32, pi32]
    lib.vmi_state_cache_slots.argtypes = [vp, i64, pi64, i64, pi32]
    lib.vmi_state_cache_refs.argtypes = [vp, i64, pi32, pi64]
    lib.vmi_state_cache_step.argtypes = [vp, i64, pi64, i64, vp, vp, vp, vp, i32, i32, vp, vp]
    lib.vmi_state_cache_attach_hologram.argtypes = [vp, i64, vp]
    lib.vmi_state_cache_cham_workspace_bytes.argtypes = [i64, i64, ctypes.POINTER(sz)]
    lib.vmi_state_cache_cham_step.argtypes = [vp, i64, pi64, i64, vp, vp, vp, vp, i32, i32, vp, vp,
                                              sz, vp]
    for name in ("create", "destroy", "new", "fork", "release", "plan", "slots", "refs", "step",
                 "attach_hologram", "cham_workspace_bytes", "cham_step"):
        getattr(lib, "vmi_state_cache_" + name).restype = i32
    lib.vmi_cham_scan_workspace_bytes.argtypes = [i64, i64, i64, ctypes.POINTER(sz)]
    lib.vmi_cham_scan_workspace_bytes.restype = i32
    lib.vmi_cham_scan_fwd.argtypes = [vp, vp, vp, vp, i32, i32, vp, vp, vp, vp, vp, i64, i64, i64,
                                      vp, sz, vp]
    lib.vmi_cham_scan_fwd.restype = i32
    lib.vmi_sssd_scan_bwd_workspace_bytes.argtypes = [i64, i64, i64, i64, ctypes.POINTER(sz)]
    lib.vmi_sssd_scan_bwd_workspace_bytes.restype = i32
    lib.vmi_sssd_scan_bwd.argtypes = [vp, vp, vp, vp, i32, i32, vp, vp, i32, vp, vp, vp, vp, vp,
                                      vp, i64, i64, i64, i64, vp, sz, vp]
    lib.vmi_sssd_scan_bwd.restype = i32
    lib.vmi_cham_step_workspace_bytes.argtypes = [i64, i64, ctypes.POINTER(sz)]
    lib.vmi_cham_step_workspace_bytes.restype = i32
    lib.vmi_cham_step_inplace.argtypes = [vp, vp, vp, vp, i32, i32, vp, vp, vp, vp, vp, i64, i64,
                                          vp, sz, vp]
    lib.vmi_cham_step_inplace.restype = i32
    lib.vmi_cham_step_fused.argtypes = [vp, i64, i32, vp, vp, vp, vp, vp, vp, i64, i64, vp, sz, vp]
    lib.vmi_cham_step_fused.restype = i32
    lib.vmi_cham_scan_fused.argtypes = [vp, i64, i32, vp, vp, vp, vp, i64, i64, i64, vp, sz, vp]
    lib.vmi_cham_scan_fused.restype = i32
    lib.vmi_cham_ns_workspace_bytes.argtypes = [i64, i64, ctypes.POINTER(sz)]
    lib.vmi_cham_ns_workspace_bytes.restype = i32
    lib.vmi_cham_ns_retraction.argtypes = [vp, vp, vp, vp, i64, i64, i32, vp, sz, vp]
    lib.vmi_cham_ns_retraction.restype = i32


def load(path: str = LIB_PATH):
    """Load (once) and return the ctypes library handle; raises RuntimeError if absent."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        _load_error = (f"verace_amd: {path} is not built; run `python verace-v1_amd/build.py` "
                       "(or __graft_entry__.build())")
        raise RuntimeError(_load_error)
    lib = ctypes.CDLL(path)
    _declare(lib)
    _lib = lib
    return lib


def available() -> bool:
    """True when the HIP library is built and loadable (does not touch the GPU)."""
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def check(status: int, what: str) -> None:
    if status != 0:
        lib = load()
        msg = lib.vmi_status_string(status).decode()
        hip = lib.vmi_last_hip_error()
        raise RuntimeError(f"verace_amd: {what} failed: {msg} (status {status}, hipError {hip})")


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
