"""GPU test of vmi_sssd_scan_fwd_noalloc (the prefill scan with its workspace in the
library's fixed 40 MiB device array instead of a caller buffer), called through the C ABI.

Bar: bit-exact against vmi_sssd_scan_fwd (the same kernels and plan; integer-exact
equality of every output and final state), on two calls in a row, the second with a smaller
input, so the second call reuses the array the first left behind; plus the fp32 path (no
workspace) and a plan whose workspace exceeds the array, which is refused with
VMI_ERR_WORKSPACE before anything is launched.
"""
import ctypes

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

VMI_ERR_WORKSPACE = 3


def _inputs(B, T, H, D, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    k = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    v = F.normalize(torch.randn(B, T, H, D, generator=g), dim=-1).to(dtype)
    d = (0.1 * torch.sigmoid(torch.randn(B, T, H, generator=g))).to(dtype)
    psi0 = torch.linalg.qr(torch.randn(B, H, D, D, generator=g))[0].contiguous()
    return q, k, v, d, psi0


def _noalloc(q, k, v, d, psi0, out, psi_out):
    from verace_amd import _lib
    lib = _lib.load()
    B, T, H, D = q.shape
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    return lib.vmi_sssd_scan_fwd_noalloc(p(q), p(k), p(v), p(d), _lib.dtype_code(q.dtype),
                                         _lib.dtype_code(d.dtype), p(psi0), p(out), p(psi_out),
                                         B, T, H, D, _lib.stream_handle(q.device))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_scan_matches_workspace_scan(device, dtype):
    from verace_amd import launch_sssd_hip_scan
    shapes = [(8, 4096, 8), (2, 512, 4)] if dtype == torch.bfloat16 else [(2, 300, 3), (1, 40, 2)]
    for i, (B, T, H) in enumerate(shapes):
        D = 128
        print(f"[case] noalloc {dtype} call {i} B{B} T{T} H{H}", flush=True)
        q, k, v, d, psi0 = (t.to(device) for t in _inputs(B, T, H, D, 30 + i, dtype))
        init = psi0 if i == 1 else None
        ref_o, ref_s = launch_sssd_hip_scan(q, k, v, d, init)
        out = torch.empty_like(q)
        psi = torch.empty(B, H, D, D, device=device)
        assert _noalloc(q, k, v, d, init, out, psi) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o) and torch.equal(psi, ref_s)


def test_noalloc_scan_refuses_a_workspace_beyond_its_array(device):
    """B4 H8 T16384 bf16 plans 8 segments with pass-A pieces: 21 transforms of 64 KiB per head,
    44 MB, above the 40 MiB array."""
    print("[case] noalloc refuses oversize plan", flush=True)
    B, T, H, D = 4, 16384, 8, 128
    q = torch.zeros(B, T, H, D, device=device, dtype=torch.bfloat16)
    d = torch.zeros(B, T, H, device=device, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    psi = torch.empty(B, H, D, D, device=device)
    assert _noalloc(q, q, q, d, None, out, psi) == VMI_ERR_WORKSPACE
