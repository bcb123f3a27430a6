"""Drop-in ``SSSDAttention`` whose scan runs on the gfx950 HIP kernels.

Same constructor, parameter names and forward signature as
``verace_v1/modules/sssd_attention.py:75-182`` (``w_q``, ``w_k``, ``w_v``, ``w_delta``,
``head_rmsnorm``, ``w_out`` are kept by name because ``state_dict`` loading and
``build_hybrid_optimizer`` look them up, ``unitary_muon.py:319-324``), and the
parameters are created in the same order, so ``torch.manual_seed(s); SSSDAttention(...)``
yields the same initial weights as the reference.

The forward is the reference's inference path (:114-136) with
``launch_sssd_triton_scan`` replaced by :func:`launch_sssd_hip_scan`:
projections, L2 normalisation, ``delta = 0.1 * sigmoid(w_delta x)`` and the
halted-token mask run as torch ops around the HIP scan; ``head_rmsnorm`` and ``w_out``
follow it.  Only device tensors that do not require grad are accepted -- the reference's
eager autograd path (:138-176) is the training path, for which no backward kernel
exists here, so such calls raise instead of silently running something else.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .hip_kernels import launch_sssd_hip_scan


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
        if not x.is_cuda:
            raise RuntimeError("verace_amd.SSSDAttention runs on a HIP device only; "
                               "move the module and inputs to the GPU")
        if x.requires_grad:
            raise RuntimeError("verace_amd.SSSDAttention has no backward kernel; the reference "
                               "trains through its eager autograd path (sssd_attention.py:138-176)")
        b, s, _ = x.shape
        q, k, v, delta = self.project(x, active_mask)
        o, psi = launch_sssd_hip_scan(q, k, v, delta, initial_state)
        o_norm = self.head_rmsnorm(o).view(b, s, self.num_heads * self.head_dim)
        output = self.w_out(o_norm)
        if return_state:
            return output, psi
        return output, None

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
        q, k, v, delta = self.project(x, active_mask)
        if s == 1:
            o = cache.step(layer, q, k, v, delta, handles)
        else:
            o, psi = launch_sssd_hip_scan(q, k, v, delta, cache.read(layer, handles))
            cache.write(layer, handles, psi)
        o_norm = self.head_rmsnorm(o).view(b, s, self.num_heads * self.head_dim)
        return self.w_out(o_norm)
