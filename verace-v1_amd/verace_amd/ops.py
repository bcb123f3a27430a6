"""The HIP launchers as torch operators (``torch.ops.verace.*``), with fake (meta) kernels and
autograd, so that FakeTensor / meta tracing and ``torch.compile(fullgraph=True)`` pass through
the scan instead of breaking the graph at a ctypes call.

Replaces, for tracing purposes, the reference's Triton launcher ``launch_sssd_triton_scan``
(``verace_v1/serving/triton_kernels.py:603-636``), which torch sees as an opaque Python call.

* ``verace::sssd_scan(q, k, v, delta, state?) -> (out, state_T)`` -- :func:`launch_sssd_hip_scan`;
  differentiable through ``verace::sssd_scan_bwd`` (:func:`launch_sssd_hip_scan_bwd`).
* ``verace::sssd_step_(q, k, v, delta, state!) -> out`` -- :func:`sssd_step_` (mutates state).
* ``verace::sssd_scan_fused(proj, H, D, mask?, rms_weight?, rms_eps, state?) -> (out, state_T)``.
* ``verace::sssd_step_fused_(proj, H, D, state!, mask?, rms_weight?, rms_eps) -> out`` --
  :func:`sssd_step_fused_` (mutates state).
* ``verace::cham_scan(q, k, v, gamma, h0_real?, h0_imag?) -> (out, h_real, h_imag)``.
* ``verace::cham_step_(q, k, v, gamma, h_real!, h_imag!, r_real!?, r_imag!?) -> out``.
* ``verace::cham_scan_fused(proj, h, mask?) -> (out, h_real, h_imag)`` -- :func:`launch_cham_hip_update_fused`.
* ``verace::cham_step_fused_(proj, h, h_real!, h_imag!, r_real!?, r_imag!?, mask?) -> out`` --
  :func:`cham_step_fused_` (mutates the states).
* ``verace::ns_retraction(h_real, h_imag, steps) -> (real, imag)``.

The eager module path calls the launchers directly (no dispatcher overhead in a decode loop);
:class:`~verace_amd.SSSDAttention` switches to these operators while ``torch.compile`` traces.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import hip_kernels as hk


@torch.library.custom_op("verace::sssd_scan", mutates_args=())
def sssd_scan(q: Tensor, k: Tensor, v: Tensor, delta: Tensor,
              state: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    return hk.launch_sssd_hip_scan(q, k, v, delta, state)


@sssd_scan.register_fake
def _sssd_scan_fake(q, k, v, delta, state=None):
    B, T, H, D = q.shape
    return torch.empty_like(q, memory_format=torch.contiguous_format), \
        q.new_empty((B, H, D, D), dtype=torch.float32)


@torch.library.custom_op("verace::sssd_scan_bwd", mutates_args=())
def sssd_scan_bwd(q: Tensor, k: Tensor, v: Tensor, delta: Tensor, psi_T: Tensor, d_out: Tensor,
                  d_psi_T: Optional[Tensor], need_d_psi0: bool
                  ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    dq, dk, dv, dd, dpsi0 = hk.launch_sssd_hip_scan_bwd(q, k, v, delta, psi_T, d_out, d_psi_T,
                                                         need_d_psi0)
    if dpsi0 is None:  # an operator returns tensors only: an empty placeholder
        dpsi0 = q.new_empty((0,), dtype=torch.float32)
    return dq, dk, dv, dd, dpsi0


@sssd_scan_bwd.register_fake
def _sssd_scan_bwd_fake(q, k, v, delta, psi_T, d_out, d_psi_T, need_d_psi0):
    B, T, H, D = q.shape
    d = delta.squeeze(-1) if delta.dim() == 4 else delta
    dpsi0 = q.new_empty((B, H, D, D) if need_d_psi0 else (0,), dtype=torch.float32)
    return (torch.empty_like(q, memory_format=torch.contiguous_format), q.new_empty(q.shape),
            q.new_empty(q.shape), torch.empty_like(d, memory_format=torch.contiguous_format), dpsi0)


def _scan_setup(ctx, inputs, output):
    q, k, v, delta, state = inputs
    _, psi = output
    ctx.save_for_backward(q, k, v, delta, psi)
    ctx.state_dtype = None if state is None else state.dtype
    ctx.k_dtype, ctx.v_dtype, ctx.delta_shape = k.dtype, v.dtype, delta.shape


def _scan_backward(ctx, d_out, d_psi):
    q, k, v, delta, psi = ctx.saved_tensors
    need0 = ctx.state_dtype is not None and ctx.needs_input_grad[4]
    if d_out is None:
        d_out = torch.zeros_like(q)
    dq, dk, dv, dd, dpsi0 = torch.ops.verace.sssd_scan_bwd(q, k, v, delta, psi, d_out, d_psi, need0)
    return (dq, dk.to(ctx.k_dtype), dv.to(ctx.v_dtype), dd.view(ctx.delta_shape),
            dpsi0.to(ctx.state_dtype) if need0 else None)


sssd_scan.register_autograd(_scan_backward, setup_context=_scan_setup)


@torch.library.custom_op("verace::sssd_step_", mutates_args=("state",))
def sssd_step_(q: Tensor, k: Tensor, v: Tensor, delta: Tensor, state: Tensor) -> Tensor:
    return hk.sssd_step_(q, k, v, delta, state)


@sssd_step_.register_fake
def _sssd_step_fake(q, k, v, delta, state):
    B, H, D, _ = state.shape
    return q.new_empty((B, 1, H, D))


@torch.library.custom_op("verace::sssd_step_fused_", mutates_args=("state",))
def sssd_step_fused_(proj: Tensor, num_heads: int, head_dim: int, state: Tensor,
                     active_mask: Optional[Tensor], rms_weight: Optional[Tensor],
                     rms_eps: Optional[float]) -> Tensor:
    return hk.sssd_step_fused_(proj, num_heads, head_dim, state, active_mask, rms_weight, rms_eps)


@sssd_step_fused_.register_fake
def _sssd_step_fused_fake(proj, num_heads, head_dim, state, active_mask, rms_weight, rms_eps):
    return proj.new_empty((proj.shape[0], 1, num_heads, head_dim))


@torch.library.custom_op("verace::sssd_scan_fused", mutates_args=())
def sssd_scan_fused(proj: Tensor, num_heads: int, head_dim: int, active_mask: Optional[Tensor],
                    rms_weight: Optional[Tensor], rms_eps: Optional[float],
                    state: Optional[Tensor]) -> Tuple[Tensor, Tensor]:
    return hk.launch_sssd_hip_scan_fused(proj, num_heads, head_dim, active_mask, rms_weight,
                                         rms_eps, state)


@sssd_scan_fused.register_fake
def _sssd_scan_fused_fake(proj, num_heads, head_dim, active_mask, rms_weight, rms_eps, state):
    B, T, _ = proj.shape
    return (proj.new_empty((B, T, num_heads, head_dim)),
            proj.new_empty((B, num_heads, head_dim, head_dim), dtype=torch.float32))


@torch.library.custom_op("verace::cham_scan", mutates_args=())
def cham_scan(q: Tensor, k: Tensor, v: Tensor, gamma: Tensor, h0_real: Optional[Tensor],
              h0_imag: Optional[Tensor]) -> Tuple[Tensor, Tensor, Tensor]:
    init = None if h0_real is None else (h0_real, h0_imag)
    out, (hr, hi) = hk.launch_cham_hip_update(q, k, v, gamma, init)
    return out, hr, hi


@cham_scan.register_fake
def _cham_scan_fake(q, k, v, gamma, h0_real, h0_imag):
    B, T, h = q.shape
    return (torch.empty_like(q, memory_format=torch.contiguous_format),
            q.new_empty((B, h, h), dtype=torch.float32), q.new_empty((B, h, h), dtype=torch.float32))


@torch.library.custom_op("verace::cham_step_", mutates_args=("h_real", "h_imag", "r_real", "r_imag"))
def cham_step_(q: Tensor, k: Tensor, v: Tensor, gamma: Tensor, h_real: Tensor, h_imag: Tensor,
               r_real: Optional[Tensor], r_imag: Optional[Tensor]) -> Tensor:
    readout = None if r_real is None else (r_real, r_imag)
    return hk.cham_step_(q, k, v, gamma, (h_real, h_imag), readout)


@cham_step_.register_fake
def _cham_step_fake(q, k, v, gamma, h_real, h_imag, r_real, r_imag):
    B, h, _ = h_real.shape
    return q.new_empty((B, 1, h))


@torch.library.custom_op("verace::cham_scan_fused", mutates_args=())
def cham_scan_fused(proj: Tensor, holographic_dim: int,
                    active_mask: Optional[Tensor]) -> Tuple[Tensor, Tensor, Tensor]:
    out, (hr, hi) = hk.launch_cham_hip_update_fused(proj, holographic_dim, active_mask)
    return out, hr, hi


@cham_scan_fused.register_fake
def _cham_scan_fused_fake(proj, holographic_dim, active_mask):
    B, T, _ = proj.shape
    h = holographic_dim
    return (proj.new_empty((B, T, h)), proj.new_empty((B, h, h), dtype=torch.float32),
            proj.new_empty((B, h, h), dtype=torch.float32))


@torch.library.custom_op("verace::cham_step_fused_",
                         mutates_args=("h_real", "h_imag", "r_real", "r_imag"))
def cham_step_fused_(proj: Tensor, holographic_dim: int, h_real: Tensor, h_imag: Tensor,
                     r_real: Optional[Tensor], r_imag: Optional[Tensor],
                     active_mask: Optional[Tensor]) -> Tensor:
    readout = None if r_real is None else (r_real, r_imag)
    return hk.cham_step_fused_(proj, holographic_dim, (h_real, h_imag), readout, active_mask)


@cham_step_fused_.register_fake
def _cham_step_fused_fake(proj, holographic_dim, h_real, h_imag, r_real, r_imag, active_mask):
    return proj.new_empty((proj.shape[0], 1, holographic_dim))


@torch.library.custom_op("verace::ns_retraction", mutates_args=())
def ns_retraction(h_real: Tensor, h_imag: Tensor, steps: int) -> Tuple[Tensor, Tensor]:
    return hk.newton_schulz_unitary_retraction(h_real, h_imag, steps)


@ns_retraction.register_fake
def _ns_fake(h_real, h_imag, steps):
    return (h_real.new_empty(h_real.shape, dtype=torch.float32),
            h_real.new_empty(h_real.shape, dtype=torch.float32))
