"""GPU parity of the fused decode step: one row of the stacked projection per item goes into
the step kernel, which normalises q, k, v, forms delta = 0.1 sigmoid(.) * mask, updates the
state in place and applies head_rmsnorm to the output (``sssd_attention.py:114-126`` and
``:177`` around the scan, at seq_len 1).

Oracle: the same steps in float64 on the host (F.normalize, sigmoid, mask, the fp64 closed-form
scan of oracle/sssd_closed.py over the steps taken, nn.RMSNorm's formula with torch's default
eps), fed the kernel's own projections.  The step computes in fp32 throughout (no f16 operand
rounding), so the bars are: state <= 1e-5 relative Frobenius error per (b, h) slice after three
steps, output <= 1e-2 for 16-bit I/O (one rounding of the output) and <= 1e-5 for fp32 I/O.
"""
import numpy as np
import pytest
import torch

from oracle import sssd_closed

pytestmark = pytest.mark.gpu

D = 128


def _rel(got, ref, slice_dims):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    red = tuple(i for i in range(got.ndim) if i not in slice_dims)
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _oracle(proj, H, mask, rms_w, eps, psi0):
    """float64 restatement of sssd_attention.py:114-126, the scan over the T steps, and :177.
    proj [B, T, n]; mask [B, T] or None; psi0 [B, H, D, D]."""
    p = proj.double().cpu().numpy()
    B, T, _ = p.shape
    HD = H * D

    def unit(x):
        x = x.reshape(B, T, H, D)
        n = np.sqrt((x ** 2).sum(-1, keepdims=True))
        return x / np.maximum(n, 1e-12)

    q, k, v = unit(p[..., :HD]), unit(p[..., HD:2 * HD]), unit(p[..., 2 * HD:3 * HD])
    d = 0.1 / (1.0 + np.exp(-p[..., 3 * HD:3 * HD + H]))
    if mask is not None:
        d = d * mask.cpu().numpy().astype(np.float64)[..., None]
    o, psi = sssd_closed.sssd_scan_closed_c(q, k, v, d, psi0.double().numpy())
    if rms_w is not None:
        ms = (o ** 2).mean(-1, keepdims=True)
        o = o / np.sqrt(ms + eps) * rms_w.double().cpu().numpy()
    return o, psi


def _steps(device, B, H, dtype, seed, with_mask, with_rms, scale, nsteps=3):
    from verace_amd.hip_kernels import rms_default_eps, sssd_step_fused_
    g = torch.Generator().manual_seed(seed)
    n = 3 * H * D + H + 5  # a row stride past the last used column
    proj = (scale * torch.randn(B, nsteps, n, generator=g)).to(dtype)
    mask = (torch.rand(B, nsteps, generator=g) > 0.25) if with_mask else None
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0].contiguous()
    w = (1.0 + 0.1 * torch.randn(D, generator=g)) if with_rms else None
    eps = rms_default_eps(dtype)
    state = psi0.to(device)
    outs = []
    for t in range(nsteps):
        m = None if mask is None else mask[:, t].to(device)
        o = sssd_step_fused_(proj[:, t:t + 1].to(device), H, D, state, m,
                             None if w is None else w.to(device), None)
        outs.append(o.float().cpu())
    torch.cuda.synchronize()
    o_ref, psi_ref = _oracle(proj, H, mask, w, eps, psi0)
    got_o = torch.cat(outs, 1).numpy()
    eo = _rel(got_o, o_ref, (0, 2))
    ep = _rel(state.cpu(), psi_ref, (0, 1))
    return eo, ep, state, psi0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,H,mask,rms,scale", [(3, 1, False, True, 1.0), (64, 8, True, True, 1.0),
                                                (5, 2, True, False, 300.0)])
def test_fused_step_matches_oracle(device, dtype, B, H, mask, rms, scale):
    print(f"[case] fused step {dtype} B={B} H={H} mask={mask} rms={rms} scale={scale}", flush=True)
    eo, ep, _, _ = _steps(device, B, H, dtype, seed=B + 7 * H, with_mask=mask, with_rms=rms,
                          scale=scale)
    bar_o = 1e-5 if dtype == torch.float32 else 1e-2
    print(f"[fused step {dtype} B{B} H{H}] rel o={eo:.2e} psi={ep:.2e}", flush=True)
    assert ep <= 1e-5 and eo <= bar_o


def test_fused_step_all_halted_keeps_state(device):
    """Every item halted (mask 0): delta = 0, R = I, the state is unchanged bit for bit and
    the output is head_rmsnorm(psi q / |q|)."""
    from verace_amd.hip_kernels import rms_default_eps, sssd_step_fused_
    print("[case] fused step all halted", flush=True)
    B, H = 4, 2
    g = torch.Generator().manual_seed(11)
    proj = torch.randn(B, 1, 3 * H * D + H, generator=g).to(torch.bfloat16)
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0].contiguous()
    w = 1.0 + 0.1 * torch.randn(D, generator=g)
    state = psi0.to(device)
    o = sssd_step_fused_(proj.to(device), H, D, state, torch.zeros(B, dtype=torch.bool, device=device),
                         w.to(device))
    torch.cuda.synchronize()
    assert torch.equal(state.cpu(), psi0)
    o_ref, _ = _oracle(proj, H, torch.zeros(B, 1, dtype=torch.bool), w, rms_default_eps(torch.bfloat16),
                       psi0)
    assert _rel(o.float().cpu().numpy(), o_ref, (0, 2)) <= 1e-2


def test_fused_step_nonfinite_token_is_identity(device):
    """A NaN or Inf in an item's k, v or delta logit makes its token the identity (the
    reference's non-finite guard, sssd_attention.py:45-71): that item's state is unchanged bit
    for bit and its output finite; the other items follow the oracle."""
    from verace_amd.hip_kernels import rms_default_eps, sssd_step_fused_
    print("[case] fused step non-finite tokens", flush=True)
    B, H = 6, 2
    HD = H * D
    g = torch.Generator().manual_seed(12)
    proj = torch.randn(B, 1, 3 * HD + H, generator=g)
    proj[0, 0, HD + 5] = float("nan")              # k of item 0, head 0
    proj[1, 0, 2 * HD + D + 3] = float("inf")      # v of item 1, head 1
    proj[2, 0, 3 * HD + 1] = float("nan")          # delta logit of item 2, head 1
    proj = proj.to(torch.bfloat16)
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0].contiguous()
    w = 1.0 + 0.1 * torch.randn(D, generator=g)
    state = psi0.to(device)
    o = sssd_step_fused_(proj.to(device), H, D, state, None, w.to(device))
    torch.cuda.synchronize()
    st = state.cpu()
    assert torch.equal(st[0, 0], psi0[0, 0]) and torch.equal(st[1, 1], psi0[1, 1])
    assert torch.equal(st[2, 1], psi0[2, 1])
    assert torch.isfinite(o).all() and torch.isfinite(st).all()
    clean = list(range(3, B))
    o_ref, psi_ref = _oracle(proj[clean], H, None, w, rms_default_eps(torch.bfloat16), psi0[clean])
    assert _rel(st[clean], psi_ref, (0, 1)) <= 1e-5
    assert _rel(o.float().cpu()[clean].numpy(), o_ref, (0, 2)) <= 1e-2


def test_module_step_fused_matches_unfused(device):
    """SSSDAttention.step_ (the decode step of the layer harness) through the fused kernel
    against the reference's op sequence (projections, F.normalize, sigmoid, mask, the unfused
    step, head_rmsnorm, w_out), both from the same state: the unfused path rounds the
    normalised q, k, v and delta to bf16, so the two agree to bf16 accuracy."""
    from verace_amd import SSSDAttention
    print("[case] module step fused vs unfused", flush=True)
    torch.manual_seed(5)
    hidden, H = 96, 2
    m = SSSDAttention(hidden_dim=hidden, num_heads=H, head_dim=D).to(device, torch.bfloat16)
    x = torch.randn(8, 1, hidden, device=device).to(torch.bfloat16)
    mask = torch.tensor([True, True, False, True, True, True, False, True], device=device)
    g = torch.Generator().manual_seed(6)
    psi0 = torch.linalg.qr(torch.randn(8, H, D, D, generator=g))[0].contiguous().to(device)
    with torch.no_grad():
        s_f, s_u = psi0.clone(), psi0.clone()
        y_f = m.step_(x, s_f, mask.view(8, 1))
        m.fuse_projections = False
        y_u = m.step_(x, s_u, mask.view(8, 1))
    torch.cuda.synchronize()
    assert _rel(y_f.float().cpu(), y_u.float().cpu(), (0,)) <= 2e-2
    assert _rel(s_f.cpu(), s_u.cpu(), (0, 1)) <= 1e-2
    assert torch.equal(s_f[2].cpu(), psi0[2].cpu()) and torch.equal(s_f[6].cpu(), psi0[6].cpu())


def test_fused_step_rejects_other_head_dims(device):
    from verace_amd import _lib
    from verace_amd.hip_kernels import sssd_step_fused_
    print("[case] fused step head_dim 64 rejected", flush=True)
    proj = torch.zeros(2, 1, 3 * 64 + 1, device=device, dtype=torch.bfloat16)
    state = torch.zeros(2, 1, 64, 64, device=device)
    with pytest.raises(RuntimeError):
        sssd_step_fused_(proj, 1, 64, state)
    lib = _lib.load()
    st = lib.vmi_sssd_step_fused(proj.data_ptr(), proj.shape[-1], 1, None, None, 0.0,
                                 state.data_ptr(), None, 2, 1, 64, None)
    assert st == 2  # VMI_ERR_UNSUPPORTED
