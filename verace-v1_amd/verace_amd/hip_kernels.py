"""Host-side launchers of the gfx950 SSSD / CHAM-NS kernels.

Mirrors the launcher API of ``verace_v1/serving/triton_kernels.py`` for this path:

* :func:`launch_sssd_hip_scan` replaces ``launch_sssd_triton_scan`` (:603-636): same
  arguments, same layouts, same return values (out in q's dtype, a fresh fp32 state).
* :func:`sssd_step_` is the opt-in in-place single-token decode step (no reference
  counterpart; the reference re-runs the forward at seq_len 1 and returns a new state).
* :func:`newton_schulz_unitary_retraction` / :func:`parallel_newton_schulz_retraction`
  replace ``cham_memory.py:21-51`` / ``:296-315`` for device tensors.

Every launcher enqueues on the current HIP stream and allocates its outputs and
workspace from torch's caching allocator.  There is no CPU path: non-device tensors,
a missing library or a failing call raise.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from . import _lib

HAS_HIP = _lib.available()


def _require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"verace_amd: {name} must be a HIP device tensor (got {t.device}); "
                           "there is no CPU path")


def _aligned(t: torch.Tensor) -> torch.Tensor:
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def launch_sssd_hip_scan(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    delta: torch.Tensor,
    initial_state: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """SSSD Cayley scan on the GPU.

    q, k, v: [batch, seq_len, num_heads, head_dim] (L2-normalised by the caller);
    delta: [batch, seq_len, num_heads]; initial_state: optional
    [batch, num_heads, head_dim, head_dim], identity when None (never modified).
    Returns (out [batch, seq_len, num_heads, head_dim] in q's dtype,
    final_state [batch, num_heads, head_dim, head_dim] float32).
    Reference: ``triton_kernels.py:603-636``; parity target ``sssd_attention.py:144-181``.
    """
    _require_device(q, "q")
    if q.dim() != 4:
        raise RuntimeError(f"verace_amd: q must be [B, T, H, D], got {tuple(q.shape)}")
    b, s, h, d_k = q.shape
    for name, t in (("k", k), ("v", v)):
        _require_device(t, name)
        if t.shape != q.shape:
            raise RuntimeError(f"verace_amd: {name} shape {tuple(t.shape)} != q shape {tuple(q.shape)}")
    _require_device(delta, "delta")
    if delta.dim() == 4 and delta.shape[-1] == 1:
        delta = delta.squeeze(-1)
    if tuple(delta.shape) != (b, s, h):
        raise RuntimeError(f"verace_amd: delta must be [B, T, H] = {(b, s, h)}, got {tuple(delta.shape)}")
    io_code = _lib.dtype_code(q.dtype)
    # the kernels read 16-byte vectors: contiguous and 16-byte aligned
    q_c = _aligned(q.contiguous())
    k_c = _aligned(k.to(q.dtype).contiguous())
    v_c = _aligned(v.to(q.dtype).contiguous())
    delta_c = delta.contiguous()
    d_code = _lib.dtype_code(delta_c.dtype)
    psi_in = None
    if initial_state is not None:
        _require_device(initial_state, "initial_state")
        if tuple(initial_state.shape) != (b, h, d_k, d_k):
            raise RuntimeError(f"verace_amd: initial_state must be {(b, h, d_k, d_k)}, "
                               f"got {tuple(initial_state.shape)}")
        psi_in = initial_state.to(torch.float32).contiguous()
    out = torch.empty_like(q_c)
    psi_out = torch.empty(b, h, d_k, d_k, device=q.device, dtype=torch.float32)
    lib = _lib.load()
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(lib.vmi_sssd_scan_workspace_bytes(b, s, h, d_k, io_code, ctypes.byref(ws_bytes)),
               "vmi_sssd_scan_workspace_bytes")
    ws = None
    if ws_bytes.value > 0:
        ws = torch.empty(ws_bytes.value, device=q.device, dtype=torch.uint8)
    _lib.check(lib.vmi_sssd_scan_fwd(_ptr(q_c), _ptr(k_c), _ptr(v_c), _ptr(delta_c), io_code,
                                     d_code, _ptr(psi_in), _ptr(out), _ptr(psi_out), b, s, h, d_k,
                                     _ptr(ws), ws_bytes.value, _lib.stream_handle(q.device)),
               "vmi_sssd_scan_fwd")
    return out, psi_out


def launch_sssd_hip_scan_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    delta: torch.Tensor,
    psi_T: torch.Tensor,
    d_out: torch.Tensor,
    d_psi_T: Optional[torch.Tensor] = None,
    need_d_psi0: bool = True,
):
    """Gradients of :func:`launch_sssd_hip_scan` (the eager autograd of
    ``sssd_attention.py:144-175`` that the reference trains through).

    q, k, v: [B, T, H, D] as given to the forward; delta: [B, T, H]; psi_T: the forward's
    final state [B, H, D, D] fp32; d_out: dL/dout [B, T, H, D]; d_psi_T: dL/dpsi_T or None.
    Returns (dq, dk, dv in q's dtype, d_delta in delta's dtype, d_psi0 fp32 or None).
    """
    _require_device(q, "q")
    if q.dim() != 4:
        raise RuntimeError(f"verace_amd: q must be [B, T, H, D], got {tuple(q.shape)}")
    b, s, h, d_k = q.shape
    for name, t in (("k", k), ("v", v), ("d_out", d_out)):
        _require_device(t, name)
        if t.shape != q.shape:
            raise RuntimeError(f"verace_amd: {name} shape {tuple(t.shape)} != q shape {tuple(q.shape)}")
    _require_device(delta, "delta")
    if delta.dim() == 4 and delta.shape[-1] == 1:
        delta = delta.squeeze(-1)
    if tuple(delta.shape) != (b, s, h):
        raise RuntimeError(f"verace_amd: delta must be [B, T, H] = {(b, s, h)}, got {tuple(delta.shape)}")
    for name, t in (("psi_T", psi_T), ("d_psi_T", d_psi_T)):
        if t is None:
            continue
        _require_device(t, name)
        if tuple(t.shape) != (b, h, d_k, d_k):
            raise RuntimeError(f"verace_amd: {name} must be {(b, h, d_k, d_k)}, got {tuple(t.shape)}")
    io_code = _lib.dtype_code(q.dtype)
    q_c = q.contiguous()
    k_c = k.to(q.dtype).contiguous()
    v_c = v.to(q.dtype).contiguous()
    delta_c = delta.contiguous()
    d_code = _lib.dtype_code(delta_c.dtype)
    do_c = d_out.contiguous()
    go_code = _lib.dtype_code(do_c.dtype)
    psi_c = psi_T.to(torch.float32).contiguous()
    dpsi_c = None if d_psi_T is None else d_psi_T.to(torch.float32).contiguous()
    dq = torch.empty_like(q_c)
    dk = torch.empty_like(q_c)
    dv = torch.empty_like(q_c)
    dd = torch.empty_like(delta_c)
    dpsi0 = torch.empty(b, h, d_k, d_k, device=q.device, dtype=torch.float32) if need_d_psi0 else None
    lib = _lib.load()
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(lib.vmi_sssd_scan_bwd_workspace_bytes(b, s, h, d_k, ctypes.byref(ws_bytes)),
               "vmi_sssd_scan_bwd_workspace_bytes")
    ws = torch.empty(ws_bytes.value, device=q.device, dtype=torch.uint8) if ws_bytes.value else None
    _lib.check(lib.vmi_sssd_scan_bwd(_ptr(q_c), _ptr(k_c), _ptr(v_c), _ptr(delta_c), io_code, d_code,
                                     _ptr(psi_c), _ptr(do_c), go_code, _ptr(dpsi_c), _ptr(dq),
                                     _ptr(dk), _ptr(dv), _ptr(dd), _ptr(dpsi0), b, s, h, d_k,
                                     _ptr(ws), ws_bytes.value, _lib.stream_handle(q.device)),
               "vmi_sssd_scan_bwd")
    return dq, dk, dv, dd, dpsi0


class SSSDScanFunction(torch.autograd.Function):
    """The scan as an autograd node: forward :func:`launch_sssd_hip_scan`, backward
    :func:`launch_sssd_hip_scan_bwd` (only the inputs and the final state are kept)."""

    @staticmethod
    def forward(ctx, q, k, v, delta, initial_state):
        if not 1 <= q.shape[-1] <= 256:  # fail here rather than in the backward
            raise RuntimeError(f"verace_amd: no backward kernel for head_dim {q.shape[-1]} "
                               "(built for 1 .. 256)")
        out, psi = launch_sssd_hip_scan(q, k, v, delta, initial_state)
        ctx.save_for_backward(q, k, v, delta, psi)
        ctx.init_dtype = None if initial_state is None else initial_state.dtype
        return out, psi

    @staticmethod
    def backward(ctx, d_out, d_psi):
        q, k, v, delta, psi = ctx.saved_tensors
        need0 = ctx.init_dtype is not None and ctx.needs_input_grad[4]
        dq, dk, dv, dd, dpsi0 = launch_sssd_hip_scan_bwd(q, k, v, delta, psi, d_out, d_psi, need0)
        return (dq, dk.to(k.dtype), dv.to(v.dtype), dd.view(delta.shape),
                None if dpsi0 is None else dpsi0.to(ctx.init_dtype))


def sssd_scan(q, k, v, delta, initial_state=None):
    """:func:`launch_sssd_hip_scan`, differentiable when autograd needs it."""
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (q, k, v, delta, initial_state)):
        return SSSDScanFunction.apply(q, k, v, delta, initial_state)
    return launch_sssd_hip_scan(q, k, v, delta, initial_state)


_RMS_EPS = {}


def rms_default_eps(dtype: torch.dtype) -> float:
    """The eps that ``nn.RMSNorm(eps=None)`` actually adds for inputs of ``dtype`` in the
    installed torch.  The documentation says ``finfo(dtype).eps``; torch 2.10 adds the eps of
    its fp32 compute type for bf16/fp16 inputs (2^-7 would change a unit-norm head's output by
    ~30 %), so it is measured once per dtype on the host: y = rms_norm(a) = a / sqrt(a^2 + eps)
    for one element a, and the nearer of the two candidates is taken."""
    if dtype not in _RMS_EPS:
        a = 2.0 ** -10
        y = float(torch.nn.functional.rms_norm(torch.tensor([a], dtype=dtype), [1]).double())
        est = max((a / y) ** 2 - a * a, 1e-30)
        cands = (torch.finfo(torch.float32).eps, torch.finfo(dtype).eps)
        _RMS_EPS[dtype] = min(cands, key=lambda e: abs(math.log(est / e)))
    return _RMS_EPS[dtype]


def fused_scan_supported(x_dtype: torch.dtype, seq_len: int, head_dim: int) -> bool:
    """Whether :func:`launch_sssd_hip_scan_fused` runs these shapes (bf16/fp16, D = 128,
    T >= 32); other shapes take the unfused ops and :func:`launch_sssd_hip_scan`."""
    return x_dtype in (torch.bfloat16, torch.float16) and head_dim == 128 and seq_len >= 32


def launch_sssd_hip_scan_fused(
    proj: torch.Tensor,
    num_heads: int,
    head_dim: int,
    active_mask: Optional[torch.Tensor] = None,
    rms_weight: Optional[torch.Tensor] = None,
    rms_eps: Optional[float] = None,
    initial_state: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The scan with the steps either side of it fused (``sssd_attention.py:114-126`` and
    ``:177``): ``proj`` [B, T, >= 3HD + H] is ``x @ [W_q; W_k; W_v; W_delta].T`` (raw); q, k,
    v are L2-normalised, ``delta = 0.1 * sigmoid(.) * active_mask`` is formed and, with
    ``rms_weight``, the output is ``head_rmsnorm(o)`` (``rms_eps`` None = the eps torch's
    ``nn.RMSNorm`` adds by default, :func:`rms_default_eps`), all inside the kernels.  Returns (out [B, T, H, D] in proj's
    dtype, final state [B, H, D, D] float32).  Shapes outside :func:`fused_scan_supported`
    raise."""
    _require_device(proj, "proj")
    if proj.dim() != 3:
        raise RuntimeError(f"verace_amd: proj must be [B, T, N], got {tuple(proj.shape)}")
    b, s, n = proj.shape
    H, D = num_heads, head_dim
    if not fused_scan_supported(proj.dtype, s, D):
        raise RuntimeError("verace_amd: fused scan needs bf16/fp16, head_dim 128 and T >= 32")
    if n < 3 * H * D + H:
        raise RuntimeError(f"verace_amd: proj has {n} columns, needs >= {3 * H * D + H}")
    if proj.stride(2) != 1 or proj.stride(1) % 8 != 0 or proj.stride(0) != s * proj.stride(1) \
            or proj.data_ptr() % 16 != 0:
        proj = _aligned(torch.nn.functional.pad(proj, (0, (-n) % 8)).contiguous())
    row = proj.stride(1)
    mask = None
    if active_mask is not None:
        _require_device(active_mask, "active_mask")
        mask = active_mask.reshape(b, s).to(torch.uint8).contiguous()
    w = None
    eps = 0.0
    if rms_weight is not None:
        _require_device(rms_weight, "rms_weight")
        w = rms_weight.to(torch.float32).contiguous()
        eps = rms_default_eps(proj.dtype) if rms_eps is None else float(rms_eps)
    psi_in = None
    if initial_state is not None:
        _require_device(initial_state, "initial_state")
        if tuple(initial_state.shape) != (b, H, D, D):
            raise RuntimeError(f"verace_amd: initial_state must be {(b, H, D, D)}, "
                               f"got {tuple(initial_state.shape)}")
        psi_in = initial_state.to(torch.float32).contiguous()
    out = torch.empty(b, s, H, D, device=proj.device, dtype=proj.dtype)
    psi_out = torch.empty(b, H, D, D, device=proj.device, dtype=torch.float32)
    lib = _lib.load()
    io_code = _lib.dtype_code(proj.dtype)
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(lib.vmi_sssd_scan_fused_workspace_bytes(b, s, H, D, io_code, ctypes.byref(ws_bytes)),
               "vmi_sssd_scan_fused_workspace_bytes")
    ws = torch.empty(ws_bytes.value, device=proj.device, dtype=torch.uint8) if ws_bytes.value else None
    _lib.check(lib.vmi_sssd_scan_fused(_ptr(proj), row, io_code, _ptr(mask), _ptr(w), eps,
                                       _ptr(psi_in), _ptr(out), _ptr(psi_out), b, s, H, D, _ptr(ws),
                                       ws_bytes.value, _lib.stream_handle(proj.device)),
               "vmi_sssd_scan_fused")
    return out, psi_out


def sssd_step_(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    delta: torch.Tensor,
    state: torch.Tensor,
) -> torch.Tensor:
    """In-place decode step: ``state <- R state``; returns ``out = state q`` in q's dtype.

    q, k, v: [B, 1, H, D] or [B, H, D]; delta: [B, 1, H], [B, H] or [B, 1, H, 1];
    state: [B, H, D, D] float32 contiguous, updated in place.  Only for callers that own
    the state: the reference never mutates ``initial_state`` (tree-search branches share
    it, ``hyper_generate.py:108-115``), so pass a copy where the state is shared.
    """
    _require_device(q, "q")
    _require_device(state, "state")
    if state.dtype != torch.float32 or not state.is_contiguous():
        raise RuntimeError("verace_amd: state must be a contiguous float32 tensor")
    B, H, D, D2 = state.shape
    if D != D2:
        raise RuntimeError(f"verace_amd: state must be [B, H, D, D], got {tuple(state.shape)}")
    io_code = _lib.dtype_code(q.dtype)
    q_c = q.reshape(B, 1, H, D).contiguous()
    k_c = k.reshape(B, 1, H, D).to(q.dtype).contiguous()
    v_c = v.reshape(B, 1, H, D).to(q.dtype).contiguous()
    delta_c = delta.reshape(B, 1, H).contiguous()
    for name, t in (("k", k_c), ("v", v_c), ("delta", delta_c)):
        _require_device(t, name)
    out = torch.empty_like(q_c)
    lib = _lib.load()
    _lib.check(lib.vmi_sssd_step_inplace(_ptr(q_c), _ptr(k_c), _ptr(v_c), _ptr(delta_c), io_code,
                                         _lib.dtype_code(delta_c.dtype), _ptr(state), _ptr(out),
                                         B, H, D, _lib.stream_handle(q.device)),
               "vmi_sssd_step_inplace")
    return out


def fused_step_supported(x_dtype: torch.dtype, head_dim: int) -> bool:
    """Whether :func:`sssd_step_fused_` runs these shapes (head_dim 128, any I/O dtype)."""
    return x_dtype in (torch.bfloat16, torch.float16, torch.float32) and head_dim == 128


def sssd_step_fused_(
    proj: torch.Tensor,
    num_heads: int,
    head_dim: int,
    state: torch.Tensor,
    active_mask: Optional[torch.Tensor] = None,
    rms_weight: Optional[torch.Tensor] = None,
    rms_eps: Optional[float] = None,
) -> torch.Tensor:
    """:func:`sssd_step_` with the steps either side of it fused (``sssd_attention.py:114-126``
    and ``:177`` at seq_len 1): ``proj`` [B, 1, >= 3HD + H] (or [B, >= 3HD + H]) is
    ``x @ [W_q; W_k; W_v; W_delta].T`` (raw); q, k, v are L2-normalised, ``delta = 0.1 *
    sigmoid(.) * active_mask`` is formed and, with ``rms_weight``, the output is
    ``head_rmsnorm(o)`` (``rms_eps`` None = the eps torch's ``nn.RMSNorm`` adds by default),
    all inside the kernel.  ``state`` [B, H, D, D] float32 contiguous is updated in place.
    Returns out [B, 1, H, D] in proj's dtype.  head_dim other than 128 raises."""
    _require_device(proj, "proj")
    _require_device(state, "state")
    H, D = num_heads, head_dim
    if not fused_step_supported(proj.dtype, D):
        raise RuntimeError("verace_amd: the fused decode step needs head_dim 128")
    if state.dtype != torch.float32 or not state.is_contiguous():
        raise RuntimeError("verace_amd: state must be a contiguous float32 tensor")
    b = proj.shape[0]
    if tuple(state.shape) != (b, H, D, D):
        raise RuntimeError(f"verace_amd: state must be {(b, H, D, D)}, got {tuple(state.shape)}")
    p2 = proj.reshape(b, proj.shape[-1])
    if proj.dim() == 3 and proj.shape[1] != 1:
        raise RuntimeError(f"verace_amd: proj must hold one token per item, got {tuple(proj.shape)}")
    if p2.shape[1] < 3 * H * D + H:
        raise RuntimeError(f"verace_amd: proj has {p2.shape[1]} columns, needs >= {3 * H * D + H}")
    if p2.stride(1) != 1:
        p2 = p2.contiguous()
    mask = None
    if active_mask is not None:
        _require_device(active_mask, "active_mask")
        mask = active_mask.reshape(b).to(torch.uint8).contiguous()
    w = None
    eps = 0.0
    if rms_weight is not None:
        _require_device(rms_weight, "rms_weight")
        w = rms_weight.to(torch.float32).contiguous()
        eps = rms_default_eps(proj.dtype) if rms_eps is None else float(rms_eps)
    out = torch.empty(b, 1, H, D, device=proj.device, dtype=proj.dtype)
    lib = _lib.load()
    _lib.check(lib.vmi_sssd_step_fused(_ptr(p2), p2.stride(0), _lib.dtype_code(proj.dtype),
                                       _ptr(mask), _ptr(w), eps, _ptr(state), _ptr(out), b, H, D,
                                       _lib.stream_handle(proj.device)),
               "vmi_sssd_step_fused")
    return out


def launch_cham_hip_update(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    gamma: torch.Tensor,
    initial_hologram: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
):
    """CHAM holographic scan on the GPU (replaces ``launch_cham_triton_update``,
    ``triton_kernels.py:639-685``; parity target ``cham_memory.py:167-238``).

    q, k, v: [batch, seq_len, holographic_dim] (h <= 1024, or a multiple of 4 up to 4096: one
    in-place step per token there); gamma: [batch, seq_len];
    initial_hologram: optional (H_real, H_imag) [batch, h, h], identity when None (never
    modified).  Returns (out [batch, seq_len, h] in q's dtype = Re(NS_3(H_t) q_t),
    (H_real, H_imag) the raw final state, float32).
    """
    _require_device(q, "q")
    if q.dim() != 3:
        raise RuntimeError(f"verace_amd: q must be [B, T, h], got {tuple(q.shape)}")
    b, s, h = q.shape
    for name, t in (("k", k), ("v", v)):
        _require_device(t, name)
        if t.shape != q.shape:
            raise RuntimeError(f"verace_amd: {name} shape {tuple(t.shape)} != q shape {tuple(q.shape)}")
    _require_device(gamma, "gamma")
    if gamma.dim() == 3 and gamma.shape[-1] == 1:
        gamma = gamma.squeeze(-1)
    if tuple(gamma.shape) != (b, s):
        raise RuntimeError(f"verace_amd: gamma must be [B, T] = {(b, s)}, got {tuple(gamma.shape)}")
    io_code = _lib.dtype_code(q.dtype)
    q_c = q.contiguous()
    k_c = k.to(q.dtype).contiguous()
    v_c = v.to(q.dtype).contiguous()
    g_c = gamma.contiguous()
    h0r = h0i = None
    if initial_hologram is not None:
        h0r, h0i = initial_hologram
        for name, t in (("H_real", h0r), ("H_imag", h0i)):
            _require_device(t, name)
            if tuple(t.shape) != (b, h, h):
                raise RuntimeError(f"verace_amd: {name} must be {(b, h, h)}, got {tuple(t.shape)}")
        h0r = h0r.to(torch.float32).contiguous()
        h0i = h0i.to(torch.float32).contiguous()
    out = torch.empty_like(q_c)
    hr = torch.empty(b, h, h, device=q.device, dtype=torch.float32)
    hi = torch.empty(b, h, h, device=q.device, dtype=torch.float32)
    lib = _lib.load()
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(lib.vmi_cham_scan_workspace_bytes(b, s, h, ctypes.byref(ws_bytes)),
               "vmi_cham_scan_workspace_bytes")
    ws = torch.empty(ws_bytes.value, device=q.device, dtype=torch.uint8) if ws_bytes.value else None
    _lib.check(lib.vmi_cham_scan_fwd(_ptr(q_c), _ptr(k_c), _ptr(v_c), _ptr(g_c), io_code,
                                     _lib.dtype_code(g_c.dtype), _ptr(h0r), _ptr(h0i), _ptr(out),
                                     _ptr(hr), _ptr(hi), b, s, h, _ptr(ws), ws_bytes.value,
                                     _lib.stream_handle(q.device)),
               "vmi_cham_scan_fwd")
    return out, (hr, hi)


def cham_fused_scan_supported(x_dtype: torch.dtype, holographic_dim: int) -> bool:
    """Whether :func:`launch_cham_hip_update_fused` runs these shapes (16-bit I/O, 128 < h <= 1024,
    h % 8 == 0); other shapes take the unfused ops and :func:`launch_cham_hip_update`."""
    h = holographic_dim
    return x_dtype in (torch.bfloat16, torch.float16) and 128 < h <= 1024 and h % 8 == 0


def launch_cham_hip_update_fused(
    proj: torch.Tensor,
    holographic_dim: int,
    active_mask: Optional[torch.Tensor] = None,
):
    """The CHAM scan from the identity with the projections' post-processing fused
    (``cham_memory.py:128-155`` before the scan): ``proj`` [B, T, >= 3h + 1] is
    ``x @ [W_q; W_k; W_v; W_gamma].T`` (raw); ``v = silu(.)``, q, k, v are L2-normalised and
    ``gamma = 0.1 * sigmoid(.) * active_mask`` inside the kernels.  Returns (out [B, T, h] in
    proj's dtype, (H_real, H_imag) the raw final state, float32), as
    :func:`launch_cham_hip_update` without an initial hologram.  Shapes outside
    :func:`cham_fused_scan_supported` raise."""
    _require_device(proj, "proj")
    if proj.dim() != 3:
        raise RuntimeError(f"verace_amd: proj must be [B, T, N], got {tuple(proj.shape)}")
    b, s, n = proj.shape
    h = holographic_dim
    if not cham_fused_scan_supported(proj.dtype, h):
        raise RuntimeError("verace_amd: the fused CHAM scan needs bf16/fp16 and 128 < h <= 1024, h % 8 == 0")
    if n < 3 * h + 1:
        raise RuntimeError(f"verace_amd: proj has {n} columns, needs >= {3 * h + 1}")
    if proj.stride(2) != 1 or proj.stride(1) % 8 != 0 or proj.stride(0) != s * proj.stride(1) \
            or proj.data_ptr() % 16 != 0:
        proj = _aligned(torch.nn.functional.pad(proj, (0, (-n) % 8)).contiguous())
    mask = None
    if active_mask is not None:
        _require_device(active_mask, "active_mask")
        mask = active_mask.reshape(b, s).to(torch.uint8).contiguous()
    out = _aligned(torch.empty(b, s, h, device=proj.device, dtype=proj.dtype))
    hr = torch.empty(b, h, h, device=proj.device, dtype=torch.float32)
    hi = torch.empty(b, h, h, device=proj.device, dtype=torch.float32)
    lib = _lib.load()
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(lib.vmi_cham_scan_workspace_bytes(b, s, h, ctypes.byref(ws_bytes)),
               "vmi_cham_scan_workspace_bytes")
    ws = torch.empty(ws_bytes.value, device=proj.device, dtype=torch.uint8) if ws_bytes.value else None
    _lib.check(lib.vmi_cham_scan_fused(_ptr(proj), proj.stride(1), _lib.dtype_code(proj.dtype),
                                       _ptr(mask), _ptr(out), _ptr(hr), _ptr(hi), b, s, h, _ptr(ws),
                                       ws_bytes.value, _lib.stream_handle(proj.device)),
               "vmi_cham_scan_fused")
    return out, (hr, hi)


def cham_step_fused_(
    proj: torch.Tensor,
    holographic_dim: int,
    hologram: Tuple[torch.Tensor, torch.Tensor],
    readout: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    active_mask: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """:func:`cham_step_` with the projections' post-processing fused (``cham_memory.py:128-155``
    at seq_len 1): ``proj`` [B, 1, >= 3h + 1] (or [B, >= 3h + 1]) is ``x @ [W_q; W_k; W_v;
    W_gamma].T`` (raw); ``v = silu(.)``, q, k, v are L2-normalised and ``gamma = 0.1 *
    sigmoid(.) * active_mask`` inside the kernel.  hologram / readout as :func:`cham_step_`,
    updated in place.  Returns ``Re(NS_3(H') q)`` [B, 1, h] in proj's dtype.  Only
    holographic_dim 1024 (the reference's default) runs fused; other sizes raise."""
    _require_device(proj, "proj")
    hr, hi = hologram
    h = holographic_dim
    for name, t in (("H_real", hr), ("H_imag", hi)):
        _require_device(t, name)
    if hr.dtype != torch.float32 or hi.dtype != torch.float32 or not hr.is_contiguous() \
            or not hi.is_contiguous() or hr.dim() != 3 or hr.shape != hi.shape:
        raise RuntimeError("verace_amd: hologram must be two contiguous float32 [B, h, h] tensors")
    B = hr.shape[0]
    if tuple(hr.shape) != (B, h, h) or proj.shape[0] != B:
        raise RuntimeError(f"verace_amd: hologram {tuple(hr.shape)} does not match proj {tuple(proj.shape)}")
    if h != 1024:
        raise RuntimeError("verace_amd: the fused CHAM step needs holographic_dim 1024")
    rr = ri = None
    if readout is not None:
        rr, ri = readout
        for name, t in (("R_real", rr), ("R_imag", ri)):
            _require_device(t, name)
            if t.dtype != torch.float32 or not t.is_contiguous() or t.shape != hr.shape:
                raise RuntimeError(f"verace_amd: {name} must be a contiguous float32 {tuple(hr.shape)} tensor")
    if proj.dim() == 3 and proj.shape[1] != 1:
        raise RuntimeError(f"verace_amd: proj must hold one token per item, got {tuple(proj.shape)}")
    p2 = proj.reshape(B, proj.shape[-1])
    if p2.shape[1] < 3 * h + 1:
        raise RuntimeError(f"verace_amd: proj has {p2.shape[1]} columns, needs >= {3 * h + 1}")
    if p2.stride(1) != 1:
        p2 = p2.contiguous()
    mask = None
    if active_mask is not None:
        _require_device(active_mask, "active_mask")
        mask = active_mask.reshape(B).to(torch.uint8).contiguous()
    out = torch.empty(B, 1, h, device=proj.device, dtype=proj.dtype)
    lib = _lib.load()
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(lib.vmi_cham_step_workspace_bytes(B, h, ctypes.byref(ws_bytes)),
               "vmi_cham_step_workspace_bytes")
    ws = torch.empty(ws_bytes.value, device=proj.device, dtype=torch.uint8) if ws_bytes.value else None
    _lib.check(lib.vmi_cham_step_fused(_ptr(p2), p2.stride(0), _lib.dtype_code(proj.dtype), _ptr(mask),
                                       _ptr(hr), _ptr(hi), _ptr(rr), _ptr(ri), _ptr(out), B, h,
                                       _ptr(ws), ws_bytes.value, _lib.stream_handle(proj.device)),
               "vmi_cham_step_fused")
    return out


def cham_step_(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    gamma: torch.Tensor,
    hologram: Tuple[torch.Tensor, torch.Tensor],
    readout: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
) -> torch.Tensor:
    """In-place CHAM decode step: ``H <- U H`` (and ``R <- U R`` for a carried readout
    state R = NS_3(H)); returns ``Re(NS_3(H') q)`` in q's dtype, [B, 1, h].

    q, k, v: [B, 1, h] or [B, h]; gamma: [B, 1], [B] or [B, 1, 1]; hologram = (H_real,
    H_imag) [B, h, h] float32 contiguous, updated in place; readout: the same shape, or None
    when H is unitary (a sequence that started from the identity: NS_3(H) = H).  Only for
    callers that own the state: the reference never mutates ``initial_hologram`` (the
    generator's branches share it), so pass copies where it is shared.  Reference: the CHAM
    forward at seq_len 1 (``cham_memory.py:117-238``) that the decode loop re-runs per token.
    h must be a multiple of 4 (<= 4096); other h up to 1024 take the general scan and a
    retraction.
    """
    hr, hi = hologram
    for name, t in (("q", q), ("H_real", hr), ("H_imag", hi)):
        _require_device(t, name)
    if hr.dtype != torch.float32 or hi.dtype != torch.float32 or not hr.is_contiguous() \
            or not hi.is_contiguous() or hr.dim() != 3 or hr.shape != hi.shape:
        raise RuntimeError("verace_amd: hologram must be two contiguous float32 [B, h, h] tensors")
    B, h, _ = hr.shape
    rr = ri = None
    if readout is not None:
        rr, ri = readout
        for name, t in (("R_real", rr), ("R_imag", ri)):
            _require_device(t, name)
            if t.dtype != torch.float32 or not t.is_contiguous() or t.shape != hr.shape:
                raise RuntimeError(f"verace_amd: {name} must be a contiguous float32 {tuple(hr.shape)} tensor")
    q_c = q.reshape(B, 1, h).contiguous()
    k_c = k.reshape(B, 1, h).to(q.dtype).contiguous()
    v_c = v.reshape(B, 1, h).to(q.dtype).contiguous()
    g_c = gamma.reshape(B).contiguous()
    for name, t in (("k", k_c), ("v", v_c), ("gamma", g_c)):
        _require_device(t, name)
    if h % 4 != 0:
        # general route: the scan from the current state (it retracts for the readout), then
        # the new raw state (and its retraction) written back in place
        out, (nr, ni) = launch_cham_hip_update(q_c, k_c, v_c, g_c.reshape(B, 1), (hr, hi))
        hr.copy_(nr)
        hi.copy_(ni)
        if readout is not None:
            r2, i2 = _ns(nr, ni, 3)
            rr.copy_(r2)
            ri.copy_(i2)
        return out
    out = torch.empty_like(q_c)
    lib = _lib.load()
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(lib.vmi_cham_step_workspace_bytes(B, h, ctypes.byref(ws_bytes)),
               "vmi_cham_step_workspace_bytes")
    ws = torch.empty(ws_bytes.value, device=q.device, dtype=torch.uint8) if ws_bytes.value else None
    _lib.check(lib.vmi_cham_step_inplace(_ptr(q_c), _ptr(k_c), _ptr(v_c), _ptr(g_c),
                                         _lib.dtype_code(q_c.dtype), _lib.dtype_code(g_c.dtype),
                                         _ptr(hr), _ptr(hi), _ptr(rr), _ptr(ri), _ptr(out), B, h,
                                         _ptr(ws), ws_bytes.value, _lib.stream_handle(q.device)),
               "vmi_cham_step_inplace")
    return out


def _ns(H_real: torch.Tensor, H_imag: torch.Tensor, steps: int) -> Tuple[torch.Tensor, torch.Tensor]:
    _require_device(H_real, "H_real")
    _require_device(H_imag, "H_imag")
    if H_real.shape != H_imag.shape or H_real.shape[-1] != H_real.shape[-2]:
        raise RuntimeError("verace_amd: H_real/H_imag must be matching [..., n, n] tensors")
    shape = H_real.shape
    n = shape[-1]
    hr = H_real.to(torch.float32).reshape(-1, n, n).contiguous()
    hi = H_imag.to(torch.float32).reshape(-1, n, n).contiguous()
    batch = hr.shape[0]
    out_r = torch.empty_like(hr)
    out_i = torch.empty_like(hi)
    lib = _lib.load()
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(lib.vmi_cham_ns_workspace_bytes(batch, n, ctypes.byref(ws_bytes)),
               "vmi_cham_ns_workspace_bytes")
    ws = torch.empty(max(ws_bytes.value, 1), device=hr.device, dtype=torch.uint8)
    _lib.check(lib.vmi_cham_ns_retraction(_ptr(hr), _ptr(hi), _ptr(out_r), _ptr(out_i), batch, n,
                                          int(steps), _ptr(ws), ws_bytes.value,
                                          _lib.stream_handle(hr.device)),
               "vmi_cham_ns_retraction")
    return out_r.reshape(shape), out_i.reshape(shape)


def newton_schulz_unitary_retraction(H_real: torch.Tensor, H_imag: torch.Tensor, steps: int = 3):
    """[b, d, d] complex NS retraction (reference ``cham_memory.py:21-51``), fp32 out."""
    return _ns(H_real, H_imag, steps)


def parallel_newton_schulz_retraction(H_real: torch.Tensor, H_imag: torch.Tensor, steps: int = 3):
    """[b, s, d, d] complex NS retraction (reference ``cham_memory.py:296-315``), fp32 out."""
    return _ns(H_real, H_imag, steps)
