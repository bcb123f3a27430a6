"""The DEC and FULL model workloads on the GPU, with every layer's SSSD state (and sampled CHAM
holograms) checked against the fp64 oracles.

Model: 12 layers, hidden 1024, H 8, D 128, CHAM h 1024, vocab 32000, bf16 weights drawn from
seed 0 (no checkpoint exists here), fixed depth (the static layer loop).  The inputs each layer's
scan and steps actually received are recorded by wrapping the fused kernels' entry points in the
model's modules (``launch_sssd_hip_scan_fused``, ``sssd_step_fused_``, ``cham_step_fused_``): the
raw bf16 projection they are handed is normalised on the host in fp64 (q, k, v L2-normalised, v
through silu first for CHAM, delta / gamma = 0.1 sigmoid(.)), as the kernels define it, and fed
to ``oracle.sssd_closed`` / ``oracle.cham_scan`` from the layer's state before the call.

* DEC: batch 64, a 512-token prefill, then 256 in-place decode steps.
  Every layer's prefill state (items 0 and 63, all heads) against fp64 from the identity (bar
  2e-2, the bf16 bar of the f16-operand chunk scan); every layer's state after the 256 steps
  against fp64 from the prefill state (bar 1e-5: the decode step is fp32); the CHAM hologram
  after the 256 steps at layers 0, 6, 11 (item 0) and layer 0 (item 63) against fp64 from the
  prefill hologram (bar 1e-5), and every layer's hologram's unitarity (item 0, 1e-4).
* FULL: B 4 x T 2048 prefill; item 0's final SSSD state of every layer
  against fp64 (bar 2e-2) and its state-norm drift (1e-4); item 0's layer-0 CHAM hologram after
  2048 tokens against fp64 (bar 3e-4: the chunked matrix-core carry rounds its operands to f16).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

L, H, D, HC = 12, 8, 128, 1024
HD = H * D


def _unit(t):
    return t / np.maximum(np.linalg.norm(t, axis=-1, keepdims=True), 1e-12)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _sssd_inputs(proj):
    """proj [T, >= 3HD + H] (the fused SSSD kernels' raw input, one item) -> q, k, v [1, T, H, D],
    delta [1, T, H] in fp64."""
    p = proj.double().cpu().numpy()
    T = p.shape[0]
    q, k, v = (_unit(p[:, i * HD:(i + 1) * HD].reshape(1, T, H, D)) for i in range(3))
    d = 0.1 * _sigmoid(p[:, 3 * HD:3 * HD + H]).reshape(1, T, H)
    return q, k, v, d


def _cham_inputs(proj):
    """proj [T, >= 3h + 1] (the fused CHAM kernels' raw input, one item) -> q, k, v [1, T, h],
    gamma [1, T] in fp64 (cham_memory.py:128-155: v through silu before its normalisation)."""
    p = proj.double().cpu().numpy()
    q = _unit(p[:, :HC])
    k = _unit(p[:, HC:2 * HC])
    vr = p[:, 2 * HC:3 * HC]
    v = _unit(vr * _sigmoid(vr))
    g = 0.1 * _sigmoid(p[:, 3 * HC])
    return q[None], k[None], v[None], g[None]


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.fixture(scope="module")
def model(device):
    from verace_amd import VeraceV1Config, VeraceV1Model
    torch.manual_seed(0)
    torch.cuda.manual_seed(0)
    cfg = VeraceV1Config(vocab_size=32000, hidden_dim=1024, num_layers=L, num_heads=H, head_dim=D,
                         chams_holographic_dim=HC)
    with torch.device(device):
        m = VeraceV1Model(cfg)
    m = m.to(torch.bfloat16).eval()
    yield m
    del m
    torch.cuda.empty_cache()


class _Recorder:
    """Wraps the fused entry points the model's modules call and keeps each call's raw
    projection rows of the selected items (cloned, still on the device)."""

    def __init__(self, monkeypatch, items):
        import verace_amd.cham_memory as cm
        import verace_amd.sssd_attention as sa
        self.items = items
        self.scan, self.sstep, self.cstep = [], [], []
        sel = torch.tensor(items)

        def rec(store, fn, proj_pos=0):
            def wrapped(*args, **kw):
                proj = args[proj_pos]
                store.append(proj.reshape(proj.shape[0], -1, proj.shape[-1])[sel.to(proj.device)].clone())
                return fn(*args, **kw)
            return wrapped
        monkeypatch.setattr(sa, "launch_sssd_hip_scan_fused", rec(self.scan, sa.launch_sssd_hip_scan_fused))
        monkeypatch.setattr(sa, "sssd_step_fused_", rec(self.sstep, sa.sssd_step_fused_))
        monkeypatch.setattr(cm, "cham_step_fused_", rec(self.cstep, cm.cham_step_fused_))


def test_dec_workload_states_match_fp64(device, model, monkeypatch):
    from oracle import cham_scan, sssd_closed
    B, P, S = 64, 512, 256
    items = [0, B - 1]
    print(f"[case] DEC: B{B} prefill {P}, {S} decode steps, {L} layers", flush=True)
    r = _Recorder(monkeypatch, items)
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, 32000, (B, P), generator=g).to(device)
    steps_ids = torch.randint(0, 32000, (S, B, 1), generator=g).to(device)
    with torch.no_grad():
        _, st = model.prefill(ids, static_depth=True)
        torch.cuda.synchronize()
        assert len(r.scan) == L, "the prefill did not take the fused SSSD scan"
        s_pre = [x.sssd[items].double().cpu().numpy() for x in st.layers]
        cham_sel = [(0, 0), (6, 0), (11, 0), (0, 1)]     # (layer, index into items)
        h_pre = {(l, i): (st.layers[l].cham[0][items[i]].double().cpu().numpy(),
                          st.layers[l].cham[1][items[i]].double().cpu().numpy()) for l, i in cham_sel}
        for t in range(S):
            model.decode_step(steps_ids[t], st, static_depth=True)
        torch.cuda.synchronize()
    assert len(r.sstep) == L * S and len(r.cstep) == L * S, "the decode did not take the fused steps"
    print("  GPU done", flush=True)
    worst = {"prefill_psi": 0.0, "decode_psi": 0.0, "decode_holo": 0.0, "unitarity": 0.0}
    for l in range(L):
        for i in range(len(items)):
            q, k, v, d = _sssd_inputs(r.scan[l][i])
            _, p64 = sssd_closed.sssd_scan_closed_c(q, k, v, d, None, want_out=False)
            worst["prefill_psi"] = max(worst["prefill_psi"], _rel(s_pre[l][i], p64[0]))
            proj = torch.cat([r.sstep[t * L + l][i] for t in range(S)], 0)
            q, k, v, d = _sssd_inputs(proj)
            _, p64 = sssd_closed.sssd_scan_closed_c(q, k, v, d, s_pre[l][i:i + 1], want_out=False)
            got = st.layers[l].sssd[items[i]].double().cpu().numpy()
            worst["decode_psi"] = max(worst["decode_psi"], _rel(got, p64[0]))
        hr = st.layers[l].cham[0][items[0]].double()
        hi = st.layers[l].cham[1][items[0]].double()
        Hc = torch.complex(hr, hi)
        eye = torch.eye(HC, dtype=torch.complex128, device=device)
        worst["unitarity"] = max(worst["unitarity"], float((Hc.conj().t() @ Hc - eye).abs().max()))
    for l, i in cham_sel:
        proj = torch.cat([r.cstep[t * L + l][i] for t in range(S)], 0)
        q, k, v, gm = _cham_inputs(proj)
        _, (sr, si) = cham_scan.cham_scan_closed(q, k, v, gm, h_pre[(l, i)][0][None], h_pre[(l, i)][1][None],
                                                 readout=False)
        got_r = st.layers[l].cham[0][items[i]].double().cpu().numpy()
        got_i = st.layers[l].cham[1][items[i]].double().cpu().numpy()
        err = _rel(np.concatenate([got_r, got_i]), np.concatenate([sr[0], si[0]]))
        worst["decode_holo"] = max(worst["decode_holo"], err)
    print("  " + " ".join(f"{k}={v:.2e}" for k, v in worst.items()), flush=True)
    assert worst["prefill_psi"] <= 2e-2
    assert worst["decode_psi"] <= 1e-5
    assert worst["decode_holo"] <= 1e-5
    assert worst["unitarity"] <= 1e-4


def test_full_workload_states_match_fp64(device, model, monkeypatch):
    from oracle import cham_scan, sssd_closed
    B, T = 4, 2048
    print(f"[case] FULL: B{B} T{T}, {L} layers", flush=True)
    r = _Recorder(monkeypatch, [0])
    import verace_amd.cham_memory as cm
    cham_proj = []
    fused = cm.launch_cham_hip_update_fused

    def rec_cham(proj, *a, **kw):
        cham_proj.append(proj[0].clone())
        return fused(proj, *a, **kw)
    monkeypatch.setattr(cm, "launch_cham_hip_update_fused", rec_cham)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 32000, (B, T), generator=g).to(device)
    with torch.no_grad():
        logits, st = model.prefill(ids, static_depth=True)
        torch.cuda.synchronize()
    assert len(r.scan) == L and len(cham_proj) == L, "the prefill did not take the fused scans"
    assert bool(torch.isfinite(logits.float()).all())
    print("  GPU done", flush=True)
    worst_psi, worst_drift = 0.0, 0.0
    for l in range(L):
        q, k, v, d = _sssd_inputs(r.scan[l][0])
        _, p64 = sssd_closed.sssd_scan_closed_c(q, k, v, d, None, want_out=False)
        got = st.layers[l].sssd[0].double().cpu().numpy()
        worst_psi = max(worst_psi, _rel(got, p64[0]))
        nrm = np.linalg.norm(got.reshape(H, -1), axis=-1) / np.sqrt(D)
        worst_drift = max(worst_drift, float(np.abs(nrm - 1).max()))
    q, k, v, gm = _cham_inputs(cham_proj[0])
    _, (sr, si) = cham_scan.cham_scan_closed(q, k, v, gm, readout=False)
    got = np.concatenate([st.layers[0].cham[0][0].double().cpu().numpy(),
                          st.layers[0].cham[1][0].double().cpu().numpy()])
    holo = _rel(got, np.concatenate([sr[0], si[0]]))
    print(f"  psi={worst_psi:.2e} drift={worst_drift:.2e} layer0_holo={holo:.2e}", flush=True)
    assert worst_psi <= 2e-2 and worst_drift <= 1e-4
    assert holo <= 3e-4
