"""Drop-in ``SSSDAttention`` whose scan runs on the gfx950 HIP kernels.

Same constructor, parameter names and forward signature as
``verace_v1/modules/sssd_attention.py:75-182`` (``w_q``, ``w_k``, ``w_v``, ``w_delta``,
``head_rmsnorm``, ``w_out`` are kept by name because ``state_dict`` loading and
``build_hybrid_optimizer`` look them up, ``unitary_muon.py:319-324``), and the
parameters are created in the same order, so ``torch.manual_seed(s); SSSDAttention(...)``
yields the same initial weights as the reference.

The forward is the reference's inference path (:114-136) with
``launch_sssd_triton_scan`` replaced by the HIP scan.  Where the fused scan runs (bf16 /
fp16, head_dim 128, T >= 32) the four projections are one GEMM against the stacked
weights and the L2 normalisation, ``delta = 0.1 * sigmoid(w_delta x)``, the halted-token
mask and ``head_rmsnorm`` happen inside the scan kernels
(:func:`launch_sssd_hip_scan_fused`); elsewhere they run as torch ops around
:func:`launch_sssd_hip_scan`.  ``w_out`` follows.  When autograd needs gradients (the
reference's training path, its eager autograd at :138-176) the projections and the
RMSNorm stay torch ops and the scan is :class:`SSSDScanFunction`, whose backward runs
on the HIP backward kernels.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops as _ops  # noqa: F401  (registers torch.ops.verace.*)
from .hip_kernels import (fused_scan_supported, fused_step_supported, launch_sssd_hip_scan,
                          launch_sssd_hip_scan_fused, sssd_scan, sssd_step_, sssd_step_fused_)


def _traced(x: torch.Tensor) -> bool:
    """True while torch.compile / FakeTensor / meta tracing runs this module: the scan then goes
    through the registered torch.ops.verace operators (fake kernels, autograd) instead of the
    ctypes launchers, so the graph does not break."""
    from torch._subclasses.fake_tensor import FakeTensor
    return torch.compiler.is_compiling() or isinstance(x, FakeTensor) or x.device.type == "meta"


class SSSDAttention(nn.Module):
    def __init__(self, hidden_dim: int = 16384, num_heads: int = 128, head_dim: int = 128,
                 spectral_dim: int = 256):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.spectral_dim = spectral_dim  # stored, unused (as in the reference, :85, :91)
        self.w_q = nn.Linear(hidden_dim, num_heads * head_dim, bias=False)
        self.w_k = nn.Linear(hidden_dim, num_heads * head_dim, bias=False)
        self.w_v = nn.Linear(hidden_dim, num_heads * head_dim, bias=False)
        self.w_delta = nn.Linear(hidden_dim, num_heads, bias=False)
        self.head_rmsnorm = nn.RMSNorm(head_dim)
        self.w_out = nn.Linear(num_heads * head_dim, hidden_dim, bias=False)
        self.fuse_projections = True  # False: always the unfused torch ops around the scan
        self._proj_key = None
        self._proj_cat = None

    def _stacked_weight(self) -> torch.Tensor:
        """[W_q; W_k; W_v; W_delta] as one [3HD + H, hidden] weight, rebuilt whenever one of
        the four changes (storage or in-place update).  Zero rows pad it to a multiple of 256:
        hipBLASLt picks a much slower kernel for N = 3HD + H (at FULL, N = 3080 ran 95.7 us
        against 66.4 us for N = 3328 on MI355X), and the scan skips the padding columns."""
        ws = (self.w_q.weight, self.w_k.weight, self.w_v.weight, self.w_delta.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype) for w in ws)
        if self._proj_key != key:
            cat = torch.cat([w.detach() for w in ws], 0)
            pad = (-cat.shape[0]) % 256
            if pad:
                cat = torch.cat([cat, cat.new_zeros(pad, cat.shape[1])], 0)
            self._proj_cat, self._proj_key = cat, key
        return self._proj_cat

    def _fused(self, x: torch.Tensor) -> bool:
        return (self.fuse_projections and fused_scan_supported(x.dtype, x.shape[1], self.head_dim)
                and all(w.dtype == x.dtype for w in (self.w_q.weight, self.w_k.weight,
                                                      self.w_v.weight, self.w_delta.weight)))

    def _scan_fused(self, x, initial_state, active_mask, rmsnorm_in_kernel: bool = True):
        """Fused projections + scan.  With ``rmsnorm_in_kernel`` the kernel applies
        head_rmsnorm too and returns its output; otherwise it returns the raw scan output o
        and the caller applies ``self.head_rmsnorm`` as a torch op (so its weight gets a
        gradient)."""
        proj = F.linear(x, self._stacked_weight())
        if not rmsnorm_in_kernel:
            return launch_sssd_hip_scan_fused(proj, self.num_heads, self.head_dim, active_mask,
                                              None, None, initial_state)
        w = self.head_rmsnorm.weight
        if w is None:
            w = torch.ones(self.head_dim, device=x.device)
        return launch_sssd_hip_scan_fused(proj, self.num_heads, self.head_dim, active_mask,
                                          w.detach(), self.head_rmsnorm.eps, initial_state)

    def project(self, x: torch.Tensor, active_mask: Optional[torch.Tensor] = None):
        """q, k, v [B,T,H,D] (L2-normalised) and delta [B,T,H] as the reference builds them
        (``sssd_attention.py:116-126``)."""
        b, s, _ = x.shape
        H, D = self.num_heads, self.head_dim
        q = F.normalize(self.w_q(x).view(b, s, H, D), p=2, dim=-1)
        k = F.normalize(self.w_k(x).view(b, s, H, D), p=2, dim=-1)
        v = F.normalize(self.w_v(x).view(b, s, H, D), p=2, dim=-1)
        delta = 0.1 * torch.sigmoid(self.w_delta(x)).view(b, s, H, 1)
        if active_mask is not None:
            while active_mask.ndim < delta.ndim:
                active_mask = active_mask.unsqueeze(-1)
            delta = delta * active_mask.to(delta.dtype)
        return q, k, v, delta.squeeze(-1)

    def forward(
        self,
        x: torch.Tensor,
        initial_state: Optional[torch.Tensor] = None,
        return_state: bool = False,
        active_mask: Optional[torch.Tensor] = None,
    ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        if _traced(x):
            return self._forward_traced(x, initial_state, return_state, active_mask)
        if not x.is_cuda:
            raise RuntimeError("verace_amd.SSSDAttention runs on a HIP device only; "
                               "move the module and inputs to the GPU")
        b, s, _ = x.shape
        # the reference's gate (sssd_attention.py:129): inputs that require grad take the
        # differentiable path
        grad = torch.is_grad_enabled() and (
            x.requires_grad or (initial_state is not None and initial_state.requires_grad))
        # Otherwise the scan is not differentiated (as the reference's GPU path, whose
        # Triton scan cuts the graph), but head_rmsnorm and w_out still are: the RMSNorm
        # runs inside the fused kernel only when its weight needs no gradient.
        rms_grad = (torch.is_grad_enabled() and self.head_rmsnorm.weight is not None
                    and self.head_rmsnorm.weight.requires_grad)
        if grad:
            q, k, v, delta = self.project(x, active_mask)
            o, psi = sssd_scan(q, k, v, delta, initial_state)
            o_norm = self.head_rmsnorm(o).view(b, s, self.num_heads * self.head_dim)
        elif self._fused(x):
            o_norm, psi = self._scan_fused(x, initial_state, active_mask,
                                           rmsnorm_in_kernel=not rms_grad)
            if rms_grad:
                o_norm = self.head_rmsnorm(o_norm)
            o_norm = o_norm.view(b, s, self.num_heads * self.head_dim)
        else:
            q, k, v, delta = self.project(x, active_mask)
            o, psi = launch_sssd_hip_scan(q, k, v, delta, initial_state)
            o_norm = self.head_rmsnorm(o).view(b, s, self.num_heads * self.head_dim)
        output = self.w_out(o_norm)
        if return_state:
            return output, psi
        return output, None

    def _forward_traced(self, x, initial_state, return_state, active_mask):
        """``forward`` on the registered operators (the same routes: differentiable scan when
        autograd needs it, the fused scan where it applies, else the unfused ops)."""
        b, s, _ = x.shape
        grad = torch.is_grad_enabled() and (
            x.requires_grad or (initial_state is not None and initial_state.requires_grad))
        rms_grad = (torch.is_grad_enabled() and self.head_rmsnorm.weight is not None
                    and self.head_rmsnorm.weight.requires_grad)
        if not grad and self._fused(x):
            ws = [w.detach() for w in (self.w_q.weight, self.w_k.weight, self.w_v.weight,
                                       self.w_delta.weight)]
            pad = (-sum(w.shape[0] for w in ws)) % 256
            if pad:
                ws.append(ws[0].new_zeros(pad, ws[0].shape[1]))
            proj = F.linear(x, torch.cat(ws, 0))
            w = None if rms_grad else self.head_rmsnorm.weight
            eps = None if w is None else self.head_rmsnorm.eps
            mask = None if active_mask is None else active_mask.reshape(b, s)
            o, psi = torch.ops.verace.sssd_scan_fused(proj, self.num_heads, self.head_dim, mask,
                                                      None if w is None else w.detach().float(),
                                                      eps, initial_state)
            if rms_grad:
                o = self.head_rmsnorm(o)
        else:
            q, k, v, delta = self.project(x, active_mask)
            o, psi = torch.ops.verace.sssd_scan(q, k, v, delta, initial_state)
            o = self.head_rmsnorm(o)
        output = self.w_out(o.reshape(b, s, self.num_heads * self.head_dim))
        return output, (psi if return_state else None)

    def step_(self, x: torch.Tensor, state: torch.Tensor,
              active_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``forward`` at seq_len 1 with the state updated in place: x [B, 1, hidden], state
        [B, H, D, D] float32 (the reference's incremental call, ``acd_engine.py:116-121`` /
        ``hyper_generate.py:59-63``, which returns a fresh state instead).  Returns the sub-layer
        output [B, 1, hidden].  Where the fused prefill would run (same dtypes, head_dim 128)
        the projections' normalisation, delta, mask and head RMSNorm run inside the step
        kernel on one stacked projection GEMM; otherwise the reference's op sequence."""
        b = x.shape[0]
        H, D = self.num_heads, self.head_dim
        if self._fused_step(x):
            rms_grad = (torch.is_grad_enabled() and self.head_rmsnorm.weight is not None
                        and self.head_rmsnorm.weight.requires_grad)
            w = None
            if not rms_grad:
                w = self.head_rmsnorm.weight
                w = torch.ones(D, device=x.device) if w is None else w.detach()
            o = sssd_step_fused_(F.linear(x, self._stacked_weight()), H, D, state, active_mask, w,
                                 self.head_rmsnorm.eps)
            if rms_grad:
                o = self.head_rmsnorm(o)
        else:
            q, k, v, delta = self.project(x, active_mask)
            o = self.head_rmsnorm(sssd_step_(q, k, v, delta, state))
        return self.w_out(o.reshape(b, 1, H * D))

    def _fused_step(self, x: torch.Tensor) -> bool:
        return (self.fuse_projections and x.shape[1] == 1
                and fused_step_supported(x.dtype, self.head_dim)
                and all(w.dtype == x.dtype for w in (self.w_q.weight, self.w_k.weight,
                                                      self.w_v.weight, self.w_delta.weight)))

    def forward_cached(self, x: torch.Tensor, cache, layer: int, handles,
                       active_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``forward`` with the per-item states kept in an :class:`SSSDStateCache`.

        Item b of ``x`` [B, T, hidden] continues sequence ``handles[b]`` at ``layer``: the
        reference passes ``initial_state=layer_states[layer][b]`` and stores the returned
        state back (``acd_engine.py:102-126``).  T = 1 is one batched step over the cache
        slots (in place, or copy-on-write for handles that share a slot); T > 1 runs the
        prefill scan from the handles' states and writes the final states back.
        """
        if not x.is_cuda:
            raise RuntimeError("verace_amd.SSSDAttention runs on a HIP device only")
        if x.requires_grad:
            raise RuntimeError("verace_amd.SSSDAttention has no backward kernel")
        b, s, _ = x.shape
        if len(handles) != b:
            raise ValueError(f"verace_amd: {len(handles)} handles for a batch of {b}")
        if self._fused(x):
            rms_grad = (torch.is_grad_enabled() and self.head_rmsnorm.weight is not None
                        and self.head_rmsnorm.weight.requires_grad)
            o_norm, psi = self._scan_fused(x, cache.read(layer, handles), active_mask,
                                           rmsnorm_in_kernel=not rms_grad)
            if rms_grad:
                o_norm = self.head_rmsnorm(o_norm)
            cache.write(layer, handles, psi)
            return self.w_out(o_norm.reshape(b, s, self.num_heads * self.head_dim))
        q, k, v, delta = self.project(x, active_mask)
        if s == 1:
            o = cache.step(layer, q, k, v, delta, handles)
        else:
            o, psi = launch_sssd_hip_scan(q, k, v, delta, cache.read(layer, handles))
            cache.write(layer, handles, psi)
        o_norm = self.head_rmsnorm(o).view(b, s, self.num_heads * self.head_dim)
        return self.w_out(o_norm)
