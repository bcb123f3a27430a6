"""The torch.ops.verace operators on the GPU: torch.library.opcheck (schema, fake kernels
against the real outputs, autograd registration), bit-equality with the launchers they wrap,
and torch.compile(fullgraph=True) through SSSDAttention and through the differentiable scan
(backend aot_eager: the graph is traced with FakeTensors and run op by op; no Triton)."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, D, dtype, device, seed=0):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype).to(device)
               for _ in range(3))
    d = (0.1 * torch.sigmoid(torch.randn(B, T, H, generator=g))).to(dtype).to(device)
    return q, k, v, d


def test_opcheck_scan_step_cham_ns(device):
    import verace_amd  # noqa: F401
    print("[case] opcheck", flush=True)
    q, k, v, d = _inputs(2, 40, 2, 64, torch.float32, device)
    st = torch.linalg.qr(torch.randn(2, 2, 64, 64))[0].contiguous().to(device)
    torch.library.opcheck(torch.ops.verace.sssd_scan.default, (q, k, v, d, st))
    torch.library.opcheck(torch.ops.verace.sssd_scan.default, (q, k, v, d, None))
    torch.library.opcheck(torch.ops.verace.sssd_step_.default,
                          (q[:, :1], k[:, :1], v[:, :1], d[:, :1], st.clone()))
    h = 32
    qc = F.normalize(torch.randn(2, 5, h), dim=-1).to(device)
    g = (0.1 * torch.rand(2, 5)).to(device)
    torch.library.opcheck(torch.ops.verace.cham_scan.default, (qc, qc, qc, g, None, None))
    H = torch.eye(h, device=device).expand(2, -1, -1).contiguous()
    torch.library.opcheck(torch.ops.verace.cham_step_.default,
                          (qc[:, :1], qc[:, :1], qc[:, :1], g[:, :1], H.clone(), torch.zeros_like(H),
                           None, None))
    torch.library.opcheck(torch.ops.verace.ns_retraction.default, (H + 0.01, H * 0, 3))
    proj = torch.randn(3, 1, 3 * 2 * 128 + 2, device=device).to(torch.bfloat16)
    st128 = torch.linalg.qr(torch.randn(3, 2, 128, 128))[0].contiguous().to(device)
    projc = torch.randn(2, 1, 3 * 1024 + 1, device=device).to(torch.bfloat16)
    Hc = torch.eye(1024, device=device).expand(2, -1, -1).contiguous()
    torch.library.opcheck(torch.ops.verace.cham_scan_fused.default,
                          (torch.randn(2, 20, 3 * 256 + 1, device=device).to(torch.bfloat16), 256, None))
    torch.library.opcheck(torch.ops.verace.cham_step_fused_.default,
                          (projc, 1024, Hc.clone(), torch.zeros_like(Hc), None, None, None))
    torch.library.opcheck(torch.ops.verace.sssd_step_fused_.default,
                          (proj, 2, 128, st128.clone(), None, torch.ones(128, device=device), None))


def test_ops_equal_launchers_and_autograd(device):
    from verace_amd import SSSDScanFunction, launch_sssd_hip_scan
    print("[case] ops == launchers", flush=True)
    q, k, v, d = _inputs(1, 70, 2, 128, torch.bfloat16, device, seed=1)
    o1, s1 = torch.ops.verace.sssd_scan(q, k, v, d, None)
    o2, s2 = launch_sssd_hip_scan(q, k, v, d)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    x = [t.float().clone().requires_grad_(True) for t in (q, k, v, d)]
    y = [t.float().clone().requires_grad_(True) for t in (q, k, v, d)]
    w = torch.randn(1, 70, 2, 128, device=device)
    o, s = torch.ops.verace.sssd_scan(*x, None)
    ((o * w).sum() + s.sum()).backward()
    o, s = SSSDScanFunction.apply(*y, None)
    ((o * w).sum() + s.sum()).backward()
    for a, b in zip(x, y):
        assert torch.equal(a.grad, b.grad)


def test_compile_fullgraph_module_and_scan(device):
    from verace_amd import SSSDAttention
    print("[case] torch.compile fullgraph", flush=True)
    torch.manual_seed(0)
    m = SSSDAttention(256, 2, 128).to(device).to(torch.bfloat16)
    x = torch.randn(2, 64, 256, device=device).bfloat16()
    with torch.no_grad():
        ref_y, ref_s = m(x, return_state=True)
        cm = torch.compile(m, fullgraph=True, backend="aot_eager")
        y, s = cm(x, return_state=True)
    torch.cuda.synchronize()
    assert torch.equal(y, ref_y) and torch.equal(s, ref_s)

    def loss_fn(q, k, v, d):
        o, st = torch.ops.verace.sssd_scan(q, k, v, d, None)
        return o.square().sum() + st.sum()

    q, k, v, d = _inputs(1, 40, 2, 64, torch.float32, device, seed=2)
    args = [t.clone().requires_grad_(True) for t in (q, k, v, d)]
    args2 = [t.clone().requires_grad_(True) for t in (q, k, v, d)]
    loss_fn(*args).backward()
    torch.compile(loss_fn, fullgraph=True, backend="aot_eager")(*args2).backward()
    for a, b in zip(args, args2):
        assert torch.allclose(a.grad, b.grad, rtol=1e-6, atol=1e-7)
