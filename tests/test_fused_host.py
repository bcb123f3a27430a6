"""Host-side pieces of the fused projection path (no GPU): the RMSNorm eps the fused
kernel is given must be the one torch's nn.RMSNorm adds (sssd_attention.py:100 builds it
with the default eps), and the stacked projection weight must follow the module's weights."""
import pytest
import torch

from verace_amd import SSSDAttention
from verace_amd.hip_kernels import fused_scan_supported, rms_default_eps


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rms_default_eps_matches_torch_rmsnorm(dtype):
    g = torch.Generator().manual_seed(0)
    D = 128
    for scale in (1.0, 1.0 / 128, 1e-3):   # small rows make eps visible
        x = (scale * torch.randn(4, D, generator=g)).to(dtype)
        y = torch.nn.RMSNorm(D).to(dtype)(x).double()
        xd = x.double()
        ref = xd / torch.sqrt((xd ** 2).mean(-1, keepdim=True) + rms_default_eps(dtype))
        tol = 2 * torch.finfo(dtype).eps
        assert torch.allclose(y, ref, rtol=tol, atol=0), (dtype, scale)


def test_stacked_weight_follows_the_module_weights():
    torch.manual_seed(0)
    m = SSSDAttention(64, 3, 128)
    w = m._stacked_weight()
    H, D = 3, 128
    assert w.shape == (3 * H * D + H + (-(3 * H * D + H)) % 256, 64)
    assert torch.equal(w[:H * D], m.w_q.weight) and torch.equal(w[3 * H * D:3 * H * D + H], m.w_delta.weight)
    assert torch.count_nonzero(w[3 * H * D + H:]) == 0
    assert m._stacked_weight() is w                  # cached while unchanged
    with torch.no_grad():
        m.w_k.weight.mul_(2.0)                       # in-place update: rebuilt
    w2 = m._stacked_weight()
    assert w2 is not w and torch.equal(w2[H * D:2 * H * D], m.w_k.weight)
    m.load_state_dict({k: v.clone() for k, v in m.state_dict().items()})
    assert torch.equal(m._stacked_weight()[2 * H * D:3 * H * D], m.w_v.weight)


def test_fused_gate():
    assert fused_scan_supported(torch.bfloat16, 32, 128)
    assert not fused_scan_supported(torch.bfloat16, 31, 128)
    assert not fused_scan_supported(torch.float32, 64, 128)
    assert not fused_scan_supported(torch.float16, 64, 64)
