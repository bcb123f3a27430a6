"""TEST INFRASTRUCTURE -- fp32 torch restatement of the reference's eager SSSD path.

Follows ``verace_v1/modules/sssd_attention.py`` op for op (same operand order for
``torch.linalg.solve``, same Blelloch association, fp32 with autocast off), on CPU.
Never imported by the product.
"""
from __future__ import annotations

import warnings
from typing import Optional, Tuple

import torch
import torch.nn.functional as F


def solve_cayley(right: torch.Tensor, left: torch.Tensor, eye: torch.Tensor) -> torch.Tensor:
    """Solve ``right @ R = left`` with the reference's non-finite guard.

    Restates ``sssd_attention.py:21-72``: probe solve under no_grad; any
    non-finite matrix has its *inputs* replaced by an (I, I) pair and is
    re-solved; a still non-finite result is zeroed (``nan_to_num``).
    """
    with torch.no_grad():
        probe = torch.linalg.solve(right, left)
        bad = ~torch.isfinite(probe)
    if not bad.any():
        return torch.linalg.solve(right, left)
    warnings.warn(
        "SSSD oracle: torch.linalg.solve returned non-finite values -- substituting a "
        "well-conditioned identity pair for those positions' INPUT",
        stacklevel=2,
    )
    bad_matrix = bad.any(dim=-1, keepdim=True).any(dim=-2, keepdim=True).expand_as(right)
    safe_right = torch.where(bad_matrix, eye.expand_as(right), right)
    safe_left = torch.where(bad_matrix, eye.expand_as(left), left)
    R = torch.linalg.solve(safe_right, safe_left)
    if not torch.isfinite(R).all():
        warnings.warn("SSSD oracle: forcing remaining non-finite entries to 0", stacklevel=2)
        R = torch.nan_to_num(R, nan=0.0, posinf=0.0, neginf=0.0)
    return R


def parallel_prefix_scan(R_seq: torch.Tensor) -> torch.Tensor:
    """Inclusive product scan, newest factor on the left (``sssd_attention.py:185-217``).

    ``P[t] = R[t] @ R[t-1] @ ... @ R[0]``; padded with identities to a power of two,
    up-sweep then down-sweep with ``P[dst] = P[dst] @ P[src]``, ``src = dst - step``.
    """
    b, h, s, d, _ = R_seq.shape
    if s == 1:
        return R_seq
    s_pad = 1 << (s - 1).bit_length()
    if s_pad > s:
        pad = torch.eye(d, dtype=R_seq.dtype).reshape(1, 1, 1, d, d).repeat(b, h, s_pad - s, 1, 1)
        R_seq = torch.cat([R_seq, pad], dim=2)
    P = R_seq.clone()
    step = 1
    while step < s_pad:
        dst = torch.arange(2 * step - 1, s_pad, 2 * step)
        src = dst - step
        P[:, :, dst] = torch.matmul(P[:, :, dst], P[:, :, src])
        step *= 2
    step = s_pad // 4
    while step > 0:
        dst = torch.arange(3 * step - 1, s_pad, 2 * step)
        src = dst - step
        P[:, :, dst] = torch.matmul(P[:, :, dst], P[:, :, src])
        step //= 2
    return P[:, :, :s]


def sssd_scan_eager(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    delta: torch.Tensor,
    initial_state: Optional[torch.Tensor] = None,
    compute_dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The eager scan of ``sssd_attention.py:144-175`` on CPU.

    q, k, v: [B, T, H, D] (any float dtype, upcast to fp32 as at :145);
    delta: [B, T, H] or [B, T, H, 1]; initial_state: [B, H, D, D] or None (identity).
    Returns (o [B, T, H, D] fp32, Psi_T [B, H, D, D] fp32) -- the values the
    reference feeds to head_rmsnorm (:177) and returns as state (:181).
    ``compute_dtype=torch.float64`` runs the same ops in fp64 (differentiable: the
    gradients the reference's training takes through this path, without fp32 rounding).
    """
    b, s, H, D = q.shape
    if delta.dim() == 3:
        delta = delta.unsqueeze(-1)
    cd = compute_dtype
    q32, k32, v32, delta32 = q.to(cd), k.to(cd), v.to(cd), delta.to(cd)
    if initial_state is not None:
        Psi_0 = initial_state.to(cd)
    else:
        Psi_0 = torch.eye(D, dtype=cd).unsqueeze(0).unsqueeze(0).repeat(b, H, 1, 1)
    eye = torch.eye(D, dtype=cd)
    kt_col = k32.transpose(1, 2).unsqueeze(-1)
    vt_row = v32.transpose(1, 2).unsqueeze(-2)
    vt_col = v32.transpose(1, 2).unsqueeze(-1)
    kt_row = k32.transpose(1, 2).unsqueeze(-2)
    A_seq = torch.matmul(kt_col, vt_row) - torch.matmul(vt_col, kt_row)
    d_seq = delta32.transpose(1, 2).unsqueeze(-1)
    scale_A = 0.5 * d_seq * A_seq
    left = eye - scale_A
    right = eye + scale_A
    R_seq = solve_cayley(right, left, eye)
    P_seq = parallel_prefix_scan(R_seq)
    Psi_seq = torch.matmul(P_seq, Psi_0.unsqueeze(2))
    q_col = q32.transpose(1, 2).unsqueeze(-1)
    o_seq = torch.matmul(Psi_seq, q_col).squeeze(-1).transpose(1, 2)
    return o_seq.contiguous(), Psi_seq[:, :, -1]


def sssd_scan_eager_chunked(q, k, v, delta, initial_state=None, chunk: int = 256):
    """Run :func:`sssd_scan_eager` over T in chunks, carrying the state.

    Chunk invariance (``scan(T1+T2) = scan(T2, init=scan(T1))``) is the contract of
    the reference's ``initial_state`` (``sssd_attention.py:147-150``; exercised by
    ``tests/test_triton_kernels.py:128-148``); it keeps the materialised
    [B, H, chunk, D, D] tensors to a bounded size.
    """
    T = q.shape[1]
    outs = []
    state = initial_state
    for t0 in range(0, T, chunk):
        o, state = sssd_scan_eager(q[:, t0:t0 + chunk], k[:, t0:t0 + chunk], v[:, t0:t0 + chunk],
                                   delta[:, t0:t0 + chunk], state)
        outs.append(o)
    return torch.cat(outs, dim=1), state


def sssd_module_forward(params: dict, x: torch.Tensor, num_heads: int, head_dim: int,
                        initial_state=None, return_state: bool = False, active_mask=None,
                        compute_dtype: torch.dtype = torch.float32):
    """Eager ``SSSDAttention.forward`` (``sssd_attention.py:103-182``) with explicit weights.

    ``params`` holds the module's state_dict entries: ``w_q.weight``, ``w_k.weight``,
    ``w_v.weight``, ``w_delta.weight``, ``head_rmsnorm.weight``, ``w_out.weight``.
    head_rmsnorm uses torch's default eps (``nn.RMSNorm(head_dim)``, :100).
    """
    b, s, _ = x.shape
    H, D = num_heads, head_dim
    q = F.normalize(F.linear(x, params["w_q.weight"]).view(b, s, H, D), p=2, dim=-1)
    k = F.normalize(F.linear(x, params["w_k.weight"]).view(b, s, H, D), p=2, dim=-1)
    v = F.normalize(F.linear(x, params["w_v.weight"]).view(b, s, H, D), p=2, dim=-1)
    delta = 0.1 * torch.sigmoid(F.linear(x, params["w_delta.weight"])).view(b, s, H, 1)
    if active_mask is not None:
        am = active_mask
        while am.ndim < delta.ndim:
            am = am.unsqueeze(-1)
        delta = delta * am.to(delta.dtype)
    o_seq, psi_T = sssd_scan_eager(q, k, v, delta, initial_state, compute_dtype=compute_dtype)
    o_norm = F.rms_norm(o_seq, (D,), params["head_rmsnorm.weight"]).reshape(b, s, H * D)
    out = F.linear(o_norm, params["w_out.weight"])
    return out, (psi_T if return_state else None)
