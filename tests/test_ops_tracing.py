"""The launchers as torch operators (verace_amd/ops.py): shapes from their fake kernels on
meta and FakeTensor inputs, and the drop-in SSSDAttention traced under FakeTensorMode on fake
HIP tensors -- no GPU is touched (these run on the CPU).  The operators' GPU behaviour,
opcheck and torch.compile(fullgraph=True) are covered by tests/test_gpu_ops.py."""
import pytest
import torch

import verace_amd  # noqa: F401  (registers torch.ops.verace.*)


def test_fake_kernels_give_reference_layouts():
    q = torch.empty(2, 40, 4, 64, device="meta", dtype=torch.bfloat16)
    d = torch.empty(2, 40, 4, device="meta", dtype=torch.bfloat16)
    o, s = torch.ops.verace.sssd_scan(q, q, q, d, None)
    assert o.shape == q.shape and o.dtype == torch.bfloat16  # out takes q's dtype
    assert s.shape == (2, 4, 64, 64) and s.dtype == torch.float32
    st = torch.empty(2, 4, 64, 64, device="meta")
    o1 = torch.ops.verace.sssd_step_(q[:, :1], q[:, :1], q[:, :1], d[:, :1], st)
    assert o1.shape == (2, 1, 4, 64)
    proj = torch.empty(2, 40, 3 * 4 * 128 + 4, device="meta", dtype=torch.bfloat16)
    o, s = torch.ops.verace.sssd_scan_fused(proj, 4, 128, None, None, None, None)
    assert o.shape == (2, 40, 4, 128) and s.shape == (2, 4, 128, 128)
    st128 = torch.empty(2, 4, 128, 128, device="meta")
    o1 = torch.ops.verace.sssd_step_fused_(proj[:, :1], 4, 128, st128, None, None, None)
    assert o1.shape == (2, 1, 4, 128) and o1.dtype == torch.bfloat16
    qc = torch.empty(3, 7, 32, device="meta")
    g = torch.empty(3, 7, device="meta")
    out, hr, hi = torch.ops.verace.cham_scan(qc, qc, qc, g, None, None)
    assert out.shape == qc.shape and hr.shape == (3, 32, 32) and hi.dtype == torch.float32
    H = torch.empty(3, 32, 32, device="meta")
    assert torch.ops.verace.cham_step_(qc[:, :1], qc[:, :1], qc[:, :1], g[:, :1], H, H.clone(),
                                       None, None).shape == (3, 1, 32)
    projc = torch.empty(3, 1, 3 * 1024 + 1, device="meta", dtype=torch.bfloat16)
    H1 = torch.empty(3, 1024, 1024, device="meta")
    o2, r2, i2 = torch.ops.verace.cham_scan_fused(projc.expand(3, 5, -1), 1024, None)
    assert o2.shape == (3, 5, 1024) and r2.shape == (3, 1024, 1024) and i2.dtype == torch.float32
    oc = torch.ops.verace.cham_step_fused_(projc, 1024, H1, H1.clone(), None, None, None)
    assert oc.shape == (3, 1, 1024) and oc.dtype == torch.bfloat16
    r, i = torch.ops.verace.ns_retraction(H, H, 3)
    assert r.shape == H.shape
    dq, dk, dv, dd, dp = torch.ops.verace.sssd_scan_bwd(q, q, q, d, st, q, None, True)
    assert dq.shape == q.shape and dd.shape == d.shape and dp.shape == st.shape


@pytest.mark.parametrize("dtype,T", [(torch.bfloat16, 64), (torch.float32, 8)])
def test_module_traces_under_fake_tensor_mode(dtype, T):
    """SSSDAttention on fake HIP tensors: the fused (bf16, T >= 32) and unfused routes give
    the reference's output and state shapes without running a kernel."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from verace_amd import SSSDAttention
    m = SSSDAttention(256, 2, 128).to(dtype)
    with FakeTensorMode(allow_non_fake_inputs=True) as mode:
        fm = mode.from_tensor
        x = torch.empty(2, T, 256, device="cuda", dtype=dtype)
        params = {n: fm(p).to("cuda") for n, p in m.named_parameters()}
        with torch.no_grad():
            out = torch.func.functional_call(m, params, (x,), {"return_state": True})
    y, st = out
    assert y.shape == (2, T, 256) and y.dtype == dtype
    assert st.shape == (2, 2, 128, 128) and st.dtype == torch.float32
