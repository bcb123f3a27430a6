"""GPU parity of the CHAM Newton-Schulz retraction against the oracle
(reference: verace_v1/modules/cham_memory.py:21-51, :296-315; its regression test
tests/test_cham.py:101-136 uses rtol 1e-5 / atol 1e-6 against an fp32 restatement)."""
import numpy as np
import pytest
import torch

from oracle import cham_ns

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch,n", [(2, 16), (2, 20), (3, 64), (2, 160), (1, 8)])
def test_ns_retraction_matches_oracle(device, batch, n):
    from verace_amd import newton_schulz_unitary_retraction
    print(f"[case] ns batch={batch} n={n}", flush=True)
    g = torch.Generator().manual_seed(n)
    # perturbation scaled so the singular values stay inside NS's convergence region
    # (0, sqrt(3)) at every n; the reference test's 0.1 is this at n = 16 (0.4 / sqrt(16))
    scale = 0.4 / n ** 0.5
    hr = torch.randn(batch, n, n, generator=g) * scale + torch.eye(n)
    hi = torch.randn(batch, n, n, generator=g) * scale
    got_r, got_i = newton_schulz_unitary_retraction(hr.to(device), hi.to(device))
    torch.cuda.synchronize()
    ref_r, ref_i = cham_ns.newton_schulz_retraction(hr.double(), hi.double())
    ref32_r, ref32_i = cham_ns.newton_schulz_retraction(hr, hi)
    # bar: the reference's own fp32-vs-fp32 tolerance, against both fp32 and fp64 oracles
    torch.testing.assert_close(got_r.cpu(), ref32_r, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(got_i.cpu(), ref32_i, rtol=1e-5, atol=1e-5)
    assert (got_r.cpu().double() - ref_r).abs().max() < 1e-5
    assert (got_i.cpu().double() - ref_i).abs().max() < 1e-5


def test_ns_4d_and_steps(device):
    from verace_amd import parallel_newton_schulz_retraction
    g = torch.Generator().manual_seed(0)
    hr = torch.randn(2, 3, 12, 12, generator=g) * 0.1 + torch.eye(12)
    hi = torch.randn(2, 3, 12, 12, generator=g) * 0.1
    for steps in (0, 1, 5):
        got_r, got_i = parallel_newton_schulz_retraction(hr.to(device), hi.to(device), steps=steps)
        ref_r, ref_i = cham_ns.newton_schulz_retraction(hr.double(), hi.double(), steps=steps)
        torch.cuda.synchronize()
        assert got_r.shape == hr.shape
        assert (got_r.cpu().double() - ref_r).abs().max() < 1e-5
        assert (got_i.cpu().double() - ref_i).abs().max() < 1e-5


def test_ns_output_is_unitary(device):
    from verace_amd import newton_schulz_unitary_retraction
    n = 32
    g = torch.Generator().manual_seed(1)
    hr = torch.randn(4, n, n, generator=g) * (0.2 / n ** 0.5) + torch.eye(n)
    hi = torch.randn(4, n, n, generator=g) * (0.2 / n ** 0.5)
    r, i = newton_schulz_unitary_retraction(hr.to(device), hi.to(device), steps=5)
    Hc = (r.cpu().double() + 1j * i.cpu().double())
    err = (Hc.conj().transpose(-1, -2) @ Hc - torch.eye(n, dtype=torch.complex128)).abs().max()
    assert float(err) < 1e-4


def test_ns_retraction_default_size(device):
    """The reference's default chams_holographic_dim (config.py:35): n = 1024, batch 2,
    against the fp64 oracle (1e-5)."""
    from verace_amd import newton_schulz_unitary_retraction
    n, batch = 1024, 2
    print(f"[case] ns batch={batch} n={n}", flush=True)
    g = torch.Generator().manual_seed(5)
    scale = 0.4 / n ** 0.5
    hr = torch.randn(batch, n, n, generator=g) * scale + torch.eye(n)
    hi = torch.randn(batch, n, n, generator=g) * scale
    got_r, got_i = newton_schulz_unitary_retraction(hr.to(device), hi.to(device))
    torch.cuda.synchronize()
    ref_r, ref_i = cham_ns.newton_schulz_retraction(hr.double(), hi.double())
    er = float((got_r.cpu().double() - ref_r).abs().max())
    ei = float((got_i.cpu().double() - ref_i).abs().max())
    rel = float(torch.sqrt(((got_r.cpu().double() - ref_r) ** 2).sum() + ((got_i.cpu().double() - ref_i) ** 2).sum())
                / torch.sqrt((ref_r ** 2).sum() + (ref_i ** 2).sum()))
    print(f"  max abs err real={er:.2e} imag={ei:.2e} rel={rel:.2e}", flush=True)
    assert er < 1e-5 and ei < 1e-5 and rel < 1e-5


@pytest.mark.parametrize("batch,n,steps", [(3, 128, 3), (2, 256, 1), (1, 384, 5), (2, 512, 3)])
def test_ns_matrix_core_route(device, batch, n, steps):
    """n a multiple of 128 runs the 16-bit matrix-core route (f16 hi + lo operands, two complex
    GEMM launches per iteration, the Gram's mirror-written tiles): against the fp64 oracle at
    the fp32 bar (1e-5), with perturbations that exercise every tile and the off-diagonal
    (mirrored) Gram tiles, and an imaginary part of the same size as the real perturbation."""
    from verace_amd import newton_schulz_unitary_retraction
    print(f"[case] ns16 batch={batch} n={n} steps={steps}", flush=True)
    g = torch.Generator().manual_seed(n + steps)
    scale = 0.4 / n ** 0.5
    hr = torch.randn(batch, n, n, generator=g) * scale + torch.eye(n)
    hi = torch.randn(batch, n, n, generator=g) * scale
    got_r, got_i = newton_schulz_unitary_retraction(hr.to(device), hi.to(device), steps=steps)
    torch.cuda.synchronize()
    ref_r, ref_i = cham_ns.newton_schulz_retraction(hr.double(), hi.double(), steps=steps)
    er = float((got_r.cpu().double() - ref_r).abs().max())
    ei = float((got_i.cpu().double() - ref_i).abs().max())
    print(f"  max abs err real={er:.2e} imag={ei:.2e}", flush=True)
    assert er < 1e-5 and ei < 1e-5
