"""GPU parity of the CHAM kernels above holographic_dim 1024 (up to 4096, h % 4 == 0): the
in-place step (vmi_cham_step_inplace / cham_step_, 4-column blocks) and the holographic scan
(vmi_cham_scan_fwd / launch_cham_hip_update), which there runs one step per token, against the
fp64 closed-form oracle (oracle/cham_scan.py, pinned to the eager restatement of
``cham_memory.py:167-238`` in tests/test_cham_oracle.py; it re-retracts every raw state for
the readout, as the reference's tiled route ``launch_cham_triton_tiled``,
``triton_kernels.py:477-597``, does).

Sizes: h = 1028 and 3000 (rows past h unused in the last row group), 2048 and 4096 (exact
tiles); unitary states without a readout state and non-unitary states with R = NS_3(H)
(h <= 2048: the fp64 retraction of a 4096-wide state is too slow for the host).  Bars: fp32
I/O 1e-5 relative Frobenius error per item (readout and state), bf16 2e-2.
"""
import numpy as np
import pytest
import torch

from oracle import cham_ns, cham_scan

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    red = tuple(range(1, got.ndim))
    num = np.sqrt(((got - ref) ** 2).sum(axis=red))
    den = np.sqrt((ref ** 2).sum(axis=red))
    return float((num / np.maximum(den, 1e-30)).max())


def _tokens(B, T, h, g, dtype):
    q = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, h, generator=g), dim=-1)
    v = torch.nn.functional.normalize(torch.nn.functional.silu(torch.randn(B, T, h, generator=g)), dim=-1)
    gam = 0.1 * torch.sigmoid(torch.randn(B, T, generator=g))
    return q.to(dtype), k.to(dtype), v.to(dtype), gam.to(dtype)


def _start(B, h, g, unitary):
    """A unitary start (QR of a random complex matrix), scaled per column when not unitary."""
    a = torch.randn(B, h, h, generator=g, dtype=torch.float64) + 1j * torch.randn(B, h, h, generator=g, dtype=torch.float64)
    u = torch.linalg.qr(a)[0]
    if not unitary:
        u = u * (1.0 + 0.05 * torch.rand(B, 1, h, generator=g, dtype=torch.float64))
    return u.real.float().contiguous(), u.imag.float().contiguous()


CASES = [(1028, True), (1028, False), (2048, True), (2048, False), (3000, True), (4096, True)]


@pytest.mark.parametrize("h,unitary", CASES)
def test_cham_step_large_h_matches_oracle(device, h, unitary):
    from verace_amd import cham_step_
    B, T = 2, 2
    print(f"[case] cham step h{h} unitary={unitary}", flush=True)
    g = torch.Generator().manual_seed(h + unitary)
    q, k, v, gam = _tokens(B, T, h, g, torch.float32)
    h0r, h0i = _start(B, h, g, unitary)
    hr, hi = h0r.to(device), h0i.to(device)
    readout = None
    if not unitary:
        rr, ri = cham_ns.newton_schulz_retraction(h0r.double(), h0i.double(), 3)
        readout = (rr.float().contiguous().to(device), ri.float().contiguous().to(device))
    outs = []
    for t in range(T):
        o = cham_step_(q[:, t:t + 1].to(device), k[:, t:t + 1].to(device), v[:, t:t + 1].to(device),
                       gam[:, t:t + 1].to(device), (hr, hi), readout)
        outs.append(o.float().cpu())
    torch.cuda.synchronize()
    out = torch.cat(outs, 1)
    ref, (sr, si) = cham_scan.cham_scan_closed(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                              gam.double().numpy(), h0r.double().numpy(), h0i.double().numpy())
    eo = _rel(out, ref)
    es = max(_rel(hr.cpu(), sr), _rel(hi.cpu(), si))
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-5 and es <= 1e-5


@pytest.mark.parametrize("h,start", [(2048, "identity"), (2048, "nonunitary"), (1028, "unitary"),
                                     (4096, "identity")])
def test_cham_scan_large_h_matches_oracle(device, h, start):
    """The scan above h = 1024 from the identity (readout from H itself), from a unitary and
    from a non-unitary initial hologram (readout state NS_3(H_0) carried in the workspace),
    fp32 I/O; the initial hologram is left unmodified."""
    from verace_amd import launch_cham_hip_update
    B, T = 2, 3
    print(f"[case] cham scan h{h} start={start}", flush=True)
    g = torch.Generator().manual_seed(7 * h + len(start))
    q, k, v, gam = _tokens(B, T, h, g, torch.float32)
    init = None
    h0r = h0i = None
    if start != "identity":
        h0r, h0i = _start(B, h, g, start == "unitary")
        init = (h0r.to(device), h0i.to(device))
    out, (hr, hi) = launch_cham_hip_update(q.to(device), k.to(device), v.to(device), gam.to(device), init)
    torch.cuda.synchronize()
    ref, (sr, si) = cham_scan.cham_scan_closed(
        q.double().numpy(), k.double().numpy(), v.double().numpy(), gam.double().numpy(),
        None if h0r is None else h0r.double().numpy(), None if h0i is None else h0i.double().numpy())
    eo = _rel(out.cpu(), ref)
    es = max(_rel(hr.cpu(), sr), _rel(hi.cpu(), si))
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-5 and es <= 1e-5
    if init is not None:
        assert torch.equal(init[0].cpu(), h0r) and torch.equal(init[1].cpu(), h0i)


def test_cham_scan_large_h_bf16_and_edges(device):
    """bf16 inputs at h = 2048 (2e-2), T = 0 (the state is H_0, no output rows), and the sizes
    the route refuses (h % 4 != 0 above 1024, h above 4096)."""
    import ctypes
    from verace_amd import launch_cham_hip_update
    from verace_amd import _lib
    B, T, h = 2, 2, 2048
    print(f"[case] cham scan h{h} bf16", flush=True)
    g = torch.Generator().manual_seed(5)
    q, k, v, gam = _tokens(B, T, h, g, torch.bfloat16)
    out, (hr, hi) = launch_cham_hip_update(q.to(device), k.to(device), v.to(device), gam.to(device))
    torch.cuda.synchronize()
    ref, (sr, si) = cham_scan.cham_scan_closed(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                                              gam.double().numpy())
    eo, es = _rel(out.float().cpu(), ref), max(_rel(hr.cpu(), sr), _rel(hi.cpu(), si))
    print(f"  rel out={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2
    h0r, h0i = _start(B, h, g, False)
    out0, (r0, i0) = launch_cham_hip_update(q[:, :0].to(device), k[:, :0].to(device), v[:, :0].to(device),
                                            gam[:, :0].to(device), (h0r.to(device), h0i.to(device)))
    torch.cuda.synchronize()
    assert out0.shape == (B, 0, h) and torch.equal(r0.cpu(), h0r) and torch.equal(i0.cpu(), h0i)
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    assert lib.vmi_cham_scan_workspace_bytes(B, T, 1026, ctypes.byref(n)) == 2  # VMI_ERR_UNSUPPORTED
    assert lib.vmi_cham_scan_workspace_bytes(B, T, 4100, ctypes.byref(n)) == 2
    assert lib.vmi_cham_step_workspace_bytes(B, 4100, ctypes.byref(n)) == 2
    assert lib.vmi_cham_step_workspace_bytes(B, 4096, ctypes.byref(n)) == 0
