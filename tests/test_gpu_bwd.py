"""GPU parity of the scan's backward (vmi_sssd_scan_bwd / SSSDScanFunction) against the
gradients of the reference's training path: fp64 autograd through the eager restatement
of ``sssd_attention.py:144-175`` (oracle/sssd_eager.py, pinned against finite
differences and an independent closed form in tests/test_bwd_algebra.py).

Bars: relative Frobenius error per gradient tensor <= 1e-5 for fp32 inputs (the fp32
bar of the forward; the kernel rebuilds the states from the fp32 final state by R_t^T),
<= 2e-2 for bf16 / fp16 inputs (gradients stored in the input type, the forward's f16
operands); the module's gradients (every weight, x and the initial state) <= 1e-4 in
fp32 (torch's fp32 GEMMs and RMSNorm around the scan).
"""
import numpy as np
import pytest
import torch

from oracle import sssd_eager

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.sqrt(((got - ref) ** 2).sum()) / max(np.sqrt((ref ** 2).sum()), 1e-30))


def _inputs(B, T, H, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    nrm = torch.nn.functional.normalize
    q = nrm(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    k = nrm(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    v = nrm(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    d = (0.1 * torch.sigmoid(torch.randn(B, T, H, generator=g))).to(dtype)
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0]
    w_o = torch.randn(B, T, H, D, generator=g)
    w_s = torch.randn(B, H, D, D, generator=g)
    return q, k, v, d, psi0, w_o, w_s


def _oracle(q, k, v, d, psi0, w_o, w_s, with_state_grad):
    a = [x.double().clone().requires_grad_(True) for x in (q, k, v, d)]
    p0 = None if psi0 is None else psi0.double().clone().requires_grad_(True)
    o, s = sssd_eager.sssd_scan_eager(*a, p0, compute_dtype=torch.float64)
    loss = (o * w_o.double()).sum()
    if with_state_grad:
        loss = loss + (s * w_s.double()).sum()
    loss.backward()
    return [x.grad for x in a] + [None if p0 is None else p0.grad]


@pytest.mark.parametrize("B,T,H,D,dtype,init,sgrad", [
    (2, 40, 2, 64, torch.float32, True, True),
    (1, 100, 2, 128, torch.float32, False, True),
    (2, 64, 4, 128, torch.bfloat16, True, True),
    (1, 1, 1, 128, torch.float32, True, False),
    (2, 33, 3, 128, torch.float16, False, False),
    (1, 50, 2, 64, torch.bfloat16, True, True),
    # B * H past a multiple of 8: whole groups of 8 heads share an XCD, the rest go in order
    (3, 40, 4, 128, torch.bfloat16, True, True),
    (2, 24, 5, 64, torch.float32, False, True),
    # head dims other than 64 / 128 (the per-token reverse pass at any T, padded inside)
    (2, 40, 2, 96, torch.float32, True, True),
    (1, 20, 3, 48, torch.float32, False, True),
    (1, 35, 1, 200, torch.bfloat16, True, True),
    (1, 12, 2, 256, torch.float32, True, True),
    (2, 9, 2, 17, torch.float32, True, True),
])
def test_scan_backward_matches_oracle(device, B, T, H, D, dtype, init, sgrad):
    from verace_amd import SSSDScanFunction
    print(f"[case] bwd B={B} T={T} H={H} D={D} {dtype} init={init} state_grad={sgrad}", flush=True)
    q, k, v, d, psi0, w_o, w_s = _inputs(B, T, H, D, seed=B * 100 + T + D, dtype=dtype)
    if not init:
        psi0 = None
    ref = _oracle(q, k, v, d, psi0, w_o, w_s, sgrad)
    a = [x.to(device).clone().requires_grad_(True) for x in (q, k, v, d)]
    p0 = None if psi0 is None else psi0.to(device).clone().requires_grad_(True)
    o, s = SSSDScanFunction.apply(*a, p0)
    loss = (o.float() * w_o.to(device)).sum()
    if sgrad:
        loss = loss + (s * w_s.to(device)).sum()
    loss.backward()
    torch.cuda.synchronize()
    got = [x.grad for x in a] + [None if p0 is None else p0.grad]
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, g_, r_ in zip(("dq", "dk", "dv", "ddelta", "dpsi0"), got, ref):
        if r_ is None:
            assert g_ is None
            continue
        e = _rel(g_.float().cpu(), r_)
        print(f"[bwd {dtype} B{B} T{T} H{H} D{D}] {name} rel {e:.2e}", flush=True)
        assert e <= tol, name


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scan_backward_long_sequence(device, dtype):
    """T = 1024: the reverse rebuild of the states stays accurate over a long sequence
    (bf16: the per-chunk gradient products take bf16 operands; the error must not grow
    with the number of chunks)."""
    from verace_amd import SSSDScanFunction
    print(f"[case] bwd long T=1024 {dtype}", flush=True)
    B, T, H, D = 1, 1024, 1, 128
    q, k, v, d, psi0, w_o, w_s = _inputs(B, T, H, D, seed=77, dtype=dtype)
    ref = _oracle(q, k, v, d, None, w_o, w_s, True)
    a = [x.to(device).clone().requires_grad_(True) for x in (q, k, v, d)]
    o, s = SSSDScanFunction.apply(*a, None)
    ((o.float() * w_o.to(device)).sum() + (s * w_s.to(device)).sum()).backward()
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, x, r_ in zip(("dq", "dk", "dv", "ddelta"), a, ref):
        e = _rel(x.grad.float().cpu(), r_)
        print(f"[bwd long {dtype}] {name} rel {e:.2e}", flush=True)
        assert e <= tol, name


def test_module_training_gradients(device):
    """SSSDAttention with inputs that require grad (the reference's training path):
    every parameter gradient, dx and d initial_state against the fp64 eager module."""
    from verace_amd import SSSDAttention
    print("[case] bwd module", flush=True)
    torch.manual_seed(0)
    hidden, H, D = 256, 2, 128
    m = SSSDAttention(hidden, H, D).to(device)
    g = torch.Generator().manual_seed(1)
    B, T = 2, 48
    x = torch.randn(B, T, hidden, generator=g)
    st0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0]
    mask = torch.rand(B, T, generator=g) > 0.2
    wy = torch.randn(B, T, hidden, generator=g)
    ws = torch.randn(B, H, D, D, generator=g)
    xd = x.to(device).requires_grad_(True)
    sd = st0.to(device).requires_grad_(True)
    y, s = m(xd, initial_state=sd, return_state=True, active_mask=mask.to(device))
    ((y * wy.to(device)).sum() + (s * ws.to(device)).sum()).backward()
    torch.cuda.synchronize()
    params = {n: p.detach().cpu().double().clone().requires_grad_(True) for n, p in m.named_parameters()}
    xr = x.double().requires_grad_(True)
    sr = st0.double().requires_grad_(True)
    yr, s_r = sssd_eager.sssd_module_forward(params, xr, H, D, sr, True, mask,
                                            compute_dtype=torch.float64)
    ((yr * wy.double()).sum() + (s_r * ws.double()).sum()).backward()
    for n, p in m.named_parameters():
        e = _rel(p.grad.cpu(), params[n].grad)
        print(f"[bwd module] {n} rel {e:.2e}", flush=True)
        assert e <= 1e-4, n
    for name, got, r_ in (("x", xd.grad, xr.grad), ("initial_state", sd.grad, sr.grad)):
        e = _rel(got.cpu(), r_)
        print(f"[bwd module] d{name} rel {e:.2e}", flush=True)
        assert e <= 1e-4, name


def test_scan_backward_empty_sequence(device):
    """T = 0: the state gradient passes through unchanged; the other gradients are empty."""
    from verace_amd import launch_sssd_hip_scan_bwd
    print("[case] bwd T=0", flush=True)
    B, H, D = 2, 3, 128
    z = torch.zeros(B, 0, H, D, device=device)
    d = torch.zeros(B, 0, H, device=device)
    psi = torch.randn(B, H, D, D, device=device)
    dpsi = torch.randn(B, H, D, D, device=device)
    dq, dk, dv, dd, dpsi0 = launch_sssd_hip_scan_bwd(z, z, z, d, psi, z, dpsi, True)
    torch.cuda.synchronize()
    assert dq.shape == (B, 0, H, D) and dd.shape == (B, 0, H)
    assert torch.equal(dpsi0, dpsi)


def test_module_rmsnorm_and_out_grads_with_detached_input(device):
    """x that needs no grad while the parameters do (frozen features): the scan is not
    differentiated (as the reference's GPU path), but head_rmsnorm and w_out still get their
    gradients on every route -- the fused one (bf16, D = 128, T >= 32) included -- equal to
    the unfused route's."""
    from verace_amd import SSSDAttention
    print("[case] rmsnorm grad with detached x", flush=True)
    torch.manual_seed(0)
    m = SSSDAttention(256, 2, 128).to(device).to(torch.bfloat16)
    with torch.no_grad():
        m.head_rmsnorm.weight.add_(0.1 * torch.randn_like(m.head_rmsnorm.weight))
    x = torch.randn(2, 64, 256, device=device).bfloat16()
    grads = {}
    for fused in (True, False):
        m.zero_grad(set_to_none=True)
        m.fuse_projections = fused
        y, _ = m(x)
        y.float().square().sum().backward()
        assert m.head_rmsnorm.weight.grad is not None and m.w_out.weight.grad is not None
        assert m.w_q.weight.grad is None  # the scan cuts the graph, as the reference's GPU path
        grads[fused] = (m.head_rmsnorm.weight.grad.float().cpu(), m.w_out.weight.grad.float().cpu())
    torch.cuda.synchronize()
    for a, b in zip(grads[True], grads[False]):
        e = _rel(a.numpy(), b.numpy())
        print(f"  fused vs unfused grad rel={e:.2e}", flush=True)
        assert e <= 2e-2


def test_backward_launcher_rejects_bad_shapes(device):
    """launch_sssd_hip_scan_bwd validates every argument before any kernel is launched."""
    from verace_amd import launch_sssd_hip_scan_bwd
    B, T, H, D = 1, 8, 2, 64
    q = torch.randn(B, T, H, D, device=device)
    d = torch.zeros(B, T, H, device=device)
    psi = torch.zeros(B, H, D, D, device=device)
    with pytest.raises(RuntimeError):
        launch_sssd_hip_scan_bwd(q, q[:, :4], q, d, psi, q)          # k shape
    with pytest.raises(RuntimeError):
        launch_sssd_hip_scan_bwd(q, q, q, d[:, :, :1], psi, q)       # delta shape
    with pytest.raises(RuntimeError):
        launch_sssd_hip_scan_bwd(q, q, q, d, psi[:, :1], q)          # psi_T shape
    with pytest.raises(RuntimeError):
        launch_sssd_hip_scan_bwd(q, q, q, d, psi, q[..., :32])       # d_out shape
    with pytest.raises(RuntimeError):
        launch_sssd_hip_scan_bwd(q, q, q, d, psi, q, psi[..., :8])   # d_psi_T shape
    with pytest.raises(RuntimeError):
        launch_sssd_hip_scan_bwd(q, q.cpu(), q, d, psi, q)           # device
