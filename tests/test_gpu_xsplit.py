"""GPU parity of the opt-in column-split prefill scan (VMI_XSPLIT=1, csrc/sssd_xsplit.hip).

Four cooperating workgroups per sequence, each owning 32 state columns; chunk factors and
partial outputs cross workgroups through rings in L2.  Checked against the fp64 closed form
(bars as for the chunk path: 2e-2 relative per (b, h) slice, state-norm drift 1e-4) and against
the default segment path on the same inputs (same f16 operand rounding, so they agree to
~1e-3 on o and ~1e-4 on the state).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sssd_closed

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, seed, dtype, ddt):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, 128, generator=g), dim=-1).to(dtype)
    k = F.normalize(torch.randn(B, T, H, 128, generator=g), dim=-1).to(dtype)
    v = F.normalize(torch.randn(B, T, H, 128, generator=g), dim=-1).to(dtype)
    d = (0.1 * torch.sigmoid(torch.randn(B, T, H, generator=g))).to(ddt)
    return q, k, v, d


def _rel(a, b, dims):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    red = tuple(i for i in range(a.ndim) if i not in dims)
    num = np.sqrt(((a - b) ** 2).sum(axis=red))
    return float((num / np.maximum(np.sqrt((b ** 2).sum(axis=red)), 1e-30)).max())


def _scan(monkeypatch, flag, q, k, v, d, psi0):
    from verace_amd import launch_sssd_hip_scan
    monkeypatch.setenv("VMI_XSPLIT", flag)
    dev = torch.device("cuda:0")
    o, p = launch_sssd_hip_scan(q.to(dev), k.to(dev), v.to(dev), d.to(dev),
                                None if psi0 is None else psi0.to(dev))
    torch.cuda.synchronize()
    return o.float().cpu(), p.cpu()


@pytest.mark.parametrize("T,dtype,ddt,with_psi0", [
    (512, torch.bfloat16, torch.bfloat16, False),
    (520, torch.bfloat16, torch.bfloat16, True),     # partial last chunk, start state
    (1024, torch.float16, torch.float32, False),
])
def test_xsplit_matches_closed_form(monkeypatch, T, dtype, ddt, with_psi0):
    B, H = 4, 8  # 32 sequences: 128 workgroups, the smallest grid the column split takes
    q, k, v, d = _inputs(B, T, H, seed=T, dtype=dtype, ddt=ddt)
    psi0 = None
    if with_psi0:
        g = torch.Generator().manual_seed(7)
        Q, _ = torch.linalg.qr(torch.randn(B, H, 128, 128, generator=g, dtype=torch.float64))
        psi0 = (3.0 * Q).float()
    ox, px = _scan(monkeypatch, "1", q, k, v, d, psi0)
    os_, ps = _scan(monkeypatch, "0", q, k, v, d, psi0)
    assert not torch.isnan(ox).any() and not torch.isnan(px).any()
    o64, p64 = sssd_closed.sssd_scan_closed_c(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                              d.float().numpy(),
                                              None if psi0 is None else psi0.double().numpy())
    eo, ep = _rel(ox, o64, (0, 2)), _rel(px, p64, (0, 1))
    n0 = (math.sqrt(128) if psi0 is None
          else np.linalg.norm(psi0.double().numpy().reshape(B, H, -1), axis=-1))
    drift = float(np.abs(np.linalg.norm(px.numpy().astype(np.float64).reshape(B, H, -1), axis=-1) / n0 - 1).max())
    print(f"xsplit T={T} {dtype}: o {eo:.2e} psi {ep:.2e} drift {drift:.2e}; "
          f"vs segment path o {_rel(ox, os_, (0, 2)):.2e} psi {_rel(px, ps, (0, 1)):.2e}")
    assert eo <= 2e-2 and ep <= 2e-2 and drift <= 1e-4
    assert _rel(ox, os_, (0, 2)) <= 5e-3 and _rel(px, ps, (0, 1)) <= 1e-3
