"""Drop-in ``ContinuousHolographicMemory`` whose holographic scan runs on the gfx950 HIP
kernels.

Same constructor, parameter names and creation order as
``verace_v1/modules/cham_memory.py:99-115`` (``w_q``, ``w_k``, ``w_v``, ``w_gamma``,
``w_out``, ``norm``), so a seeded construction gives the reference's initial weights and its
``state_dict`` loads unchanged.  The forward is the reference's (``:117-238``): the
projections, ``F.normalize`` of q and k, ``F.normalize(F.silu(w_v x))``,
``gamma = 0.1 * sigmoid(w_gamma x) * active_mask`` as torch ops, then the scan
(:func:`launch_cham_hip_update`: the exact Cayley recurrence on the raw state and the
Newton-Schulz readout ``Re(NS_3(H_t) q_t)``), then ``norm(w_out(.))``.  The raw final state
``(H_real, H_imag)`` is returned, never retracted.

:meth:`step_` is the opt-in in-place single-token step for callers that own the state (a
decode loop): the reference re-runs the forward at seq_len 1 and returns a fresh state.  At
holographic_dim 1024 it runs the projections as one GEMM on the stacked weights and lets the
step kernel form silu(v), the normalisations and gamma (:func:`cham_step_fused_`); the forward
does the same for a scan from the identity with 16-bit inputs and 128 < h <= 1024
(:func:`launch_cham_hip_update_fused`).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .hip_kernels import (cham_fused_scan_supported, cham_step_, cham_step_fused_,
                          launch_cham_hip_update, launch_cham_hip_update_fused)


class ContinuousHolographicMemory(nn.Module):
    def __init__(self, hidden_dim: int = 16384, holographic_dim: int = 1024):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.holographic_dim = holographic_dim
        self.w_q = nn.Linear(hidden_dim, holographic_dim, bias=False)
        self.w_k = nn.Linear(hidden_dim, holographic_dim, bias=False)
        self.w_v = nn.Linear(hidden_dim, holographic_dim, bias=False)
        self.w_gamma = nn.Linear(hidden_dim, 1, bias=False)
        self.w_out = nn.Linear(holographic_dim, hidden_dim, bias=False)
        self.norm = nn.RMSNorm(hidden_dim)
        self.fuse_projections = True  # False: the decode step always takes the unfused ops
        self._proj_key = None
        self._proj_cat = None

    def _stacked_weight(self) -> torch.Tensor:
        """[W_q; W_k; W_v; W_gamma] as one [3h + 1, hidden] weight, rebuilt whenever one of the
        four changes (storage or in-place update), zero rows padding it to a multiple of 256 (the
        GEMM library's kernel choice for odd N is much slower)."""
        ws = (self.w_q.weight, self.w_k.weight, self.w_v.weight, self.w_gamma.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype) for w in ws)
        if self._proj_key != key:
            cat = torch.cat([w.detach() for w in ws], 0)
            pad = (-cat.shape[0]) % 256
            if pad:
                cat = torch.cat([cat, cat.new_zeros(pad, cat.shape[1])], 0)
            self._proj_cat, self._proj_key = cat, key
        return self._proj_cat

    def _fused_scan(self, x: torch.Tensor) -> bool:
        return (self.fuse_projections and cham_fused_scan_supported(x.dtype, self.holographic_dim)
                and all(w.dtype == x.dtype for w in (self.w_q.weight, self.w_k.weight,
                                                      self.w_v.weight, self.w_gamma.weight)))

    def _fused_step(self, x: torch.Tensor) -> bool:
        return (self.fuse_projections and x.shape[1] == 1 and self.holographic_dim == 1024
                and x.dtype in (torch.bfloat16, torch.float16, torch.float32)
                and all(w.dtype == x.dtype for w in (self.w_q.weight, self.w_k.weight,
                                                      self.w_v.weight, self.w_gamma.weight)))

    def project(self, x: torch.Tensor, active_mask: Optional[torch.Tensor] = None):
        """q, k, v [B, T, h] and gamma [B, T] as the reference builds them (:128-155)."""
        q = F.normalize(self.w_q(x), p=2, dim=-1)
        k = F.normalize(self.w_k(x), p=2, dim=-1)
        v = F.normalize(F.silu(self.w_v(x)), p=2, dim=-1)
        gamma = 0.1 * torch.sigmoid(self.w_gamma(x))
        if active_mask is not None:
            am = active_mask
            while am.ndim < gamma.ndim:
                am = am.unsqueeze(-1)
            gamma = gamma * am.to(gamma.dtype)
        return q, k, v, gamma.squeeze(-1)

    def forward(
        self,
        x: torch.Tensor,
        initial_hologram: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
        active_mask: Optional[torch.Tensor] = None,
    ) -> Tuple[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
        if not x.is_cuda:
            raise RuntimeError("verace_amd.ContinuousHolographicMemory runs on a HIP device only")
        if torch.is_grad_enabled() and x.requires_grad:
            raise RuntimeError("verace_amd.ContinuousHolographicMemory has no backward kernel "
                               "(the CHAM scan is inference-only here); run under torch.no_grad()")
        if initial_hologram is None and self._fused_scan(x):
            # one projection GEMM; silu, the normalisations and gamma in the scan's kernels
            rec, hologram = launch_cham_hip_update_fused(F.linear(x, self._stacked_weight()),
                                                         self.holographic_dim, active_mask)
        else:
            q, k, v, gamma = self.project(x, active_mask)
            rec, hologram = launch_cham_hip_update(q, k, v, gamma, initial_hologram)
        y = self.norm(self.w_out(rec.to(self.w_out.weight.dtype)))
        return y, hologram

    def step_(self, x: torch.Tensor, hologram: Tuple[torch.Tensor, torch.Tensor],
              readout: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
              active_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One token per item, x [B, 1, hidden], with the raw state (H_real, H_imag)
        [B, h, h] float32 updated in place.  ``readout`` is the readout state
        R = NS_3(H) carried beside H (updated in place too) when H is not unitary; None
        when H came from the identity start (then NS_3(H) = H).  Returns y [B, 1, hidden]."""
        if self._fused_step(x):  # one projection GEMM; normalisation and gamma in the kernel
            rec = cham_step_fused_(F.linear(x, self._stacked_weight()), self.holographic_dim,
                                   hologram, readout, active_mask)
        else:
            q, k, v, gamma = self.project(x, active_mask)
            rec = cham_step_(q, k, v, gamma, hologram, readout)
        return self.norm(self.w_out(rec.to(self.w_out.weight.dtype)))
