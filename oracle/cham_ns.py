"""TEST INFRASTRUCTURE -- restatement of the CHAM Newton-Schulz unitary retraction.

``newton_schulz_retraction`` follows ``verace_v1/modules/cham_memory.py:21-51`` (3-D
[b, d, d]) and ``:296-315`` (4-D [b, s, d, d]): ``steps`` iterations of
H <- 0.5 H (3I - H^H H) in real arithmetic, both halves from the pre-update H.
Works on torch tensors of any float dtype (fp64 for ground truth).  Never imported by
the product.
"""
from __future__ import annotations

import torch


def newton_schulz_retraction(H_real: torch.Tensor, H_imag: torch.Tensor, steps: int = 3):
    d = H_real.shape[-1]
    eye = torch.eye(d, dtype=H_real.dtype, device=H_real.device)
    for _ in range(steps):
        HH_r = H_real.transpose(-1, -2) @ H_real + H_imag.transpose(-1, -2) @ H_imag
        HH_i = H_real.transpose(-1, -2) @ H_imag - H_imag.transpose(-1, -2) @ H_real
        diff_r = 3.0 * eye - HH_r
        diff_i = -HH_i
        H_real, H_imag = (
            0.5 * (H_real @ diff_r - H_imag @ diff_i),
            0.5 * (H_real @ diff_i + H_imag @ diff_r),
        )
    return H_real, H_imag
