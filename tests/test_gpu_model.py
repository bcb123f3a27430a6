"""GPU parity of the layer harness (verace_amd.backbone, restating backbone.py:21-210 and the
ACDE loop acd_engine.py:36-167) against outputs of the reference model itself
(tests/golden/model_golden.npz, written by tests/golden/make_golden_model.py in the
development container; see tests/test_model_host.py for the seeded weights).

* CPU config (VeraceV1Model seed 0, hidden 256, 2 layers, H 4, D 64,
  vocab 32000, CHAM 1024, fp32, batch 2 x seq 128, ACDE): every SSSD call the reference made
  (per layer and batch item) rerun through verace_amd.SSSDAttention in fp32 at the 1e-5 bar;
  every CHAM call through ContinuousHolographicMemory (h = 1024, the wide route) at 1e-5; the
  whole model's logits (first 64 vocabulary entries of every token, per-token sums) and its
  final SSSD states.
* tiny model (hidden 64, 4 layers, CHAM 32, halting threshold 0.0474 so that some tokens halt
  after layer 2): ACDE logits, depth counts, per-item layer states, static-depth logits, and
  the one-token incremental step both through forward(layer_states=...) and through the
  batched in-place decode (prefill / decode_step).

Bars: fp32 relative Frobenius error <= 1e-5 per SSSD / CHAM call and per state; <= 1e-4 for
logits after the whole stack (torch's fp32 GEMMs, RMSNorms and the M-CMoE GEMM formulation
add rounding of their own around the scans).
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

from test_model_host import cpu_config_model, tiny_model  # noqa: E402


def _rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.sqrt(((got - ref) ** 2).sum()) / max(np.sqrt((ref ** 2).sum()), 1e-30))


@pytest.fixture(scope="module")
def cpu_model(device):
    m, z = cpu_config_model()
    return m.to(device).eval(), z


def _sssd_state_fp64(attn, x, init):
    """Final state of SSSDAttention on x by the fp64 closed-form oracle (projections in fp64)."""
    import torch.nn.functional as F
    from oracle import sssd_closed
    W = {n: p.detach().double().cpu() for n, p in attn.state_dict().items()}
    x = torch.from_numpy(np.asarray(x)).double()
    H, D = attn.num_heads, attn.head_dim
    q = F.normalize(F.linear(x, W["w_q.weight"]).view(x.shape[0], -1, H, D), dim=-1)
    k = F.normalize(F.linear(x, W["w_k.weight"]).view(x.shape[0], -1, H, D), dim=-1)
    v = F.normalize(F.linear(x, W["w_v.weight"]).view(x.shape[0], -1, H, D), dim=-1)
    dl = 0.1 * torch.sigmoid(F.linear(x, W["w_delta.weight"]))
    _, p64 = sssd_closed.sssd_scan_closed_c(q.numpy(), k.numpy(), v.numpy(), dl.numpy(),
                                            None if init is None else np.asarray(init, np.float64))
    return p64


def test_cpu_config_sssd_layers(device, cpu_model):
    """Outputs against the reference's own outputs at the fp32 bar (1e-5).  The final state
    is held to 1e-5 against the fp64 closed form.  Against the reference's fp32 eager state,
    the bar widens by that state's own distance from fp64 (1.2e-5 here, from its LU solves and
    Blelloch products), as the SURVEY's adjudication rule prescribes where fp32 eager drifts."""
    m, z = cpu_model
    n = int(z["cpu/sssd_calls"])
    assert n == 4  # 2 layers x 2 batch items (ACDE runs the layers per item)
    for j in range(n):
        layer = int(z[f"cpu/sssd/{j}/layer"])
        print(f"[case] cpu-config SSSD call {j} layer {layer}", flush=True)
        x = torch.from_numpy(z[f"cpu/sssd/{j}/x"]).to(device)
        init_np = z[f"cpu/sssd/{j}/init"] if f"cpu/sssd/{j}/init" in z.files else None
        init = None if init_np is None else torch.from_numpy(init_np).to(device)
        with torch.no_grad():
            y, st = m.layers[layer].sssd_attn(x, initial_state=init, return_state=True)
        torch.cuda.synchronize()
        p64 = _sssd_state_fp64(m.layers[layer].sssd_attn, z[f"cpu/sssd/{j}/x"], init_np)
        ref_st = z[f"cpu/sssd/{j}/state"]
        ey = _rel(y.cpu(), z[f"cpu/sssd/{j}/y"])
        es64, es_ref, ref_own = _rel(st.cpu(), p64), _rel(st.cpu(), ref_st), _rel(ref_st, p64)
        print(f"  rel y={ey:.2e}; state vs fp64={es64:.2e}, vs reference={es_ref:.2e} "
              f"(reference vs fp64 {ref_own:.2e})", flush=True)
        assert ey <= 1e-5 and es64 <= 1e-5 and es_ref <= 1e-5 + ref_own


def _cham_state_fp64(cham, x):
    """Final raw hologram of ContinuousHolographicMemory on x (one item) by the fp64 closed
    form (projections in fp64, cham_memory.py:128-155; no readout)."""
    import torch.nn.functional as F
    from oracle import cham_scan
    W = {n: p.detach().double().cpu() for n, p in cham.state_dict().items()}
    x = torch.from_numpy(np.asarray(x)).double()
    q = F.normalize(F.linear(x, W["w_q.weight"]), dim=-1)
    k = F.normalize(F.linear(x, W["w_k.weight"]), dim=-1)
    v = F.normalize(F.silu(F.linear(x, W["w_v.weight"])), dim=-1)
    g = 0.1 * torch.sigmoid(F.linear(x, W["w_gamma.weight"])).squeeze(-1)
    _, (hr, hi) = cham_scan.cham_scan_closed(q.numpy(), k.numpy(), v.numpy(), g.numpy(),
                                             readout=False)
    return hr, hi


def test_cpu_config_cham_layers(device, cpu_model):
    """Outputs and the raw state's leading 32 x 32 block against the reference's own (1e-5).
    The state norm is held to 1e-5 against the fp64 closed form.  Against the reference's fp32
    eager norm, the bar widens by that norm's own distance from fp64 (its solves, prefix scan
    and products in fp32; the reference's comment puts its unitarity drift after 256 tokens
    at ~1e-4)."""
    m, z = cpu_model
    n = int(z["cpu/cham_calls"])
    assert n == 4
    for j in range(n):
        layer = int(z[f"cpu/cham/{j}/layer"])
        print(f"[case] cpu-config CHAM call {j} layer {layer} (h = 1024)", flush=True)
        x = torch.from_numpy(z[f"cpu/cham/{j}/x"]).to(device)
        with torch.no_grad():
            y, (hr, hi) = m.layers[layer].cham_memory(x)
        torch.cuda.synchronize()
        ey = _rel(y.cpu(), z[f"cpu/cham/{j}/y"])
        er = _rel(hr[0, :32, :32].cpu(), z[f"cpu/cham/{j}/h_real/slice"])
        hr64, _ = _cham_state_fp64(m.layers[layer].cham_memory, z[f"cpu/cham/{j}/x"])
        n64 = float(np.linalg.norm(hr64))
        n_ref = float(z[f"cpu/cham/{j}/h_real/norm"])
        nr = float(hr.double().norm())
        en64, en_ref, ref_own = abs(nr - n64) / n64, abs(nr - n_ref) / n_ref, abs(n_ref - n64) / n64
        es64 = _rel(hr[0].double().cpu(), hr64[0])
        print(f"  rel y={ey:.2e} state slice={er:.2e}; state vs fp64={es64:.2e}; ||H_real|| vs "
              f"fp64={en64:.2e}, vs reference={en_ref:.2e} (reference vs fp64 {ref_own:.2e})",
              flush=True)
        assert ey <= 1e-5 and er <= 1e-5 and es64 <= 1e-5 and en64 <= 1e-5
        assert en_ref <= 1e-5 + ref_own


def test_cpu_config_model_logits(device, cpu_model):
    m, z = cpu_model
    print("[case] cpu-config model logits (ACDE)", flush=True)
    ids = torch.from_numpy(z["cpu/input_ids"]).to(device)
    with torch.no_grad():
        logits, depth, states = m(ids, return_layer_states=True)
    torch.cuda.synchronize()
    lg = logits.double().cpu().numpy()
    e_head = _rel(lg[..., :64], z["cpu/logits_head"])
    e_sum = _rel(lg.sum(-1), z["cpu/logits_sum"])
    e_sq = _rel((lg ** 2).sum(-1), z["cpu/logits_sq"])
    agree = float((lg.argmax(-1) == z["cpu/logits_argmax"]).mean())
    st = np.stack([np.stack([s[0].cpu().numpy() for s in layer]) for layer in states])
    e_st = _rel(st, z["cpu/sssd_states"])
    print(f"  logits head={e_head:.2e} sum={e_sum:.2e} sq={e_sq:.2e} argmax agree={agree:.4f} "
          f"states={e_st:.2e}", flush=True)
    assert np.array_equal(depth.cpu().numpy(), z["cpu/depth"])
    # final SSSD states: 1e-5 against the fp64 closed form run on the reference's per-call
    # inputs (the same calls, in the same order); against the reference's fp32 eager states
    # the bar widens by their own distance from fp64 (see test_cpu_config_sssd_layers)
    p64 = np.stack([np.stack([_sssd_state_fp64(m.layers[l].sssd_attn, z[f"cpu/sssd/{2 * l + i}/x"],
                                               None)[0] for i in range(2)]) for l in range(2)])
    p64 = p64.reshape(z["cpu/sssd_states"].shape)
    assert all(int(z[f"cpu/sssd/{2 * l + i}/layer"]) == l for l in range(2) for i in range(2))
    e64, ref_own = _rel(st, p64), _rel(z["cpu/sssd_states"], p64)
    print(f"  states vs fp64={e64:.2e} (reference vs fp64 {ref_own:.2e})", flush=True)
    assert e_head <= 1e-4 and e_sum <= 1e-4 and e_sq <= 1e-4
    assert e64 <= 1e-5 and e_st <= 1e-5 + ref_own
    assert agree >= 0.99


@pytest.fixture(scope="module")
def tiny(device):
    m, z, _, _ = tiny_model()
    return m.to(device).eval(), z


def _check_states(states, z, tag, none_is_identity=False):
    """Largest relative error over the per-layer, per-item (sssd, (H_real, H_imag)) states.
    Where the reference holds None (a layer that never ran for an item), ours is None too, or
    the identity when ``none_is_identity`` (the batched decode keeps explicit states)."""
    worst = 0.0
    for l, layer in enumerate(states):
        for i, s in enumerate(layer):
            key = f"tiny/{tag}/{l}/{i}/sssd"
            if key not in z.files:
                if none_is_identity:
                    D, h = s[0].shape[-1], s[1][0].shape[-1]
                    assert torch.equal(s[0][0].cpu(), torch.eye(D).expand_as(s[0][0].cpu()))
                    assert torch.equal(s[1][0][0].cpu(), torch.eye(h))
                else:
                    assert s is None, (tag, l, i)
                continue
            worst = max(worst, _rel(s[0].cpu(), z[key]),
                        _rel(s[1][0].cpu(), z[f"tiny/{tag}/{l}/{i}/cham_real"]),
                        _rel(s[1][1].cpu(), z[f"tiny/{tag}/{l}/{i}/cham_imag"]))
    return worst


def test_tiny_model_acde_static_and_step(device, tiny):
    m, z = tiny
    print("[case] tiny model ACDE / static / incremental step", flush=True)
    ids = torch.from_numpy(z["tiny/input_ids"]).to(device)
    nxt = torch.from_numpy(z["tiny/next_ids"]).to(device)
    with torch.no_grad():
        logits, depth, states = m(ids, return_layer_states=True)
        logits1, depth1, states1 = m(nxt, layer_states=states, return_layer_states=True)
        logits_s, _ = m(ids, use_adaptive_depth=False)
    torch.cuda.synchronize()
    e = _rel(logits.cpu(), z["tiny/logits"])
    e1 = _rel(logits1.cpu(), z["tiny/logits_step"])
    es = _rel(logits_s.cpu(), z["tiny/logits_static"])
    ed = float(np.abs(depth.cpu().numpy() - z["tiny/depth"]).max())
    ed1 = float(np.abs(depth1.cpu().numpy() - z["tiny/depth_step"]).max())
    w0, w1 = _check_states(states, z, "states"), _check_states(states1, z, "states_step")
    # depth = N(t) + R(t) (acd_engine.py:67-79): a token still active after all 4 layers
    # counts 4 plus its remainder (> 4); one that halted earlier counts at most 4
    halted = float((z["tiny/depth"] <= 4 + 1e-6).mean())
    print(f"  logits acde={e:.2e} step={e1:.2e} static={es:.2e} depth err={ed:.1e}/{ed1:.1e} "
          f"states={w0:.2e}/{w1:.2e} (fraction of tokens halting early {halted:.2f})", flush=True)
    assert 0.0 < halted < 1.0  # the per-item gathered path ran
    assert e <= 1e-5 and e1 <= 1e-5 and es <= 1e-5 and ed <= 1e-5 and ed1 <= 1e-5
    assert w0 <= 1e-5 and w1 <= 1e-5


def test_tiny_model_batched_inplace_decode(device, tiny):
    """prefill + decode_step (one SSSD and one CHAM step launch per layer, states in place)
    gives the reference's incremental step."""
    m, z = tiny
    print("[case] tiny model prefill + decode_step", flush=True)
    ids = torch.from_numpy(z["tiny/input_ids"]).to(device)
    nxt = torch.from_numpy(z["tiny/next_ids"]).to(device)
    with torch.no_grad():
        logits, st = m.prefill(ids)
        logits1 = m.decode_step(nxt, st)
    torch.cuda.synchronize()
    e = _rel(logits.cpu(), z["tiny/logits"])
    e1 = _rel(logits1.cpu(), z["tiny/logits_step"])
    w1 = _check_states(st.to_layer_states(), z, "states_step", none_is_identity=True)
    print(f"  logits prefill={e:.2e} step={e1:.2e} states={w1:.2e}", flush=True)
    assert e <= 1e-5 and e1 <= 1e-5 and w1 <= 1e-5


def test_full_config_layer(device):
    """One layer of the FULL config (hidden 1024, H 8, D 128, CHAM h 1024,
    M-CMoE rank 32 x 64 components, random-init bf16 weights, B4 x T2048, identity start; layer
    index 1, so no block-residual snapshot) through the HIP path (backbone.py:53-101), checked
    against the fp64 oracles on slices small enough for the host:
      * SSSD sub-layer, item 0, all 2048 tokens and 8 heads: q, k, v, delta from the captured
        sub-layer input in fp32 (sssd_attention.py:114-126), the fp64 closed-form scan, head
        RMSNorm and w_out; module output and final state within 2e-2 (bf16 with fp32 state),
        every item's state norm within 1e-4 of sqrt(D);
      * CHAM sub-layer, item 0, first 64 tokens (cham_memory.py:128-243 on the fp64 closed
        form with the matrix-free NS_3 readout): output within 2e-2; every item's final raw
        hologram keeps ||H||_F = sqrt(h) within 1e-4 (unitary factors from the identity).
    """
    import torch.nn.functional as F
    from oracle import cham_scan, sssd_closed
    from verace_amd.backbone import VeraceV1Config, VeraceV1Layer

    print("[case] FULL-config layer B4 T2048 hidden 1024 bf16", flush=True)
    torch.manual_seed(0)
    cfg = VeraceV1Config(vocab_size=32000)
    layer = VeraceV1Layer(1, cfg).to(device=device, dtype=torch.bfloat16).eval()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 2048, cfg.hidden_dim, generator=g).to(device=device, dtype=torch.bfloat16)
    cap = {}

    def grab(name):
        def fn(mod, args, kwargs, out):
            cap[name] = (args[0].detach(), out)
        return fn

    hooks = [layer.sssd_attn.register_forward_hook(grab("sssd"), with_kwargs=True),
             layer.cham_memory.register_forward_hook(grab("cham"), with_kwargs=True)]
    with torch.no_grad():
        h_out, _, psi, (hr, hi) = layer(x)
    torch.cuda.synchronize()
    for hk in hooks:
        hk.remove()
    assert torch.isfinite(h_out).all()

    # ---- SSSD sub-layer, item 0
    a = layer.sssd_attn
    xs, (ys, _) = cap["sssd"]
    W = {n: p.detach().float().cpu() for n, p in a.state_dict().items()}
    x0 = xs[0:1].float().cpu()
    H, D = cfg.num_heads, cfg.head_dim
    q = F.normalize(F.linear(x0, W["w_q.weight"]).view(1, -1, H, D), dim=-1)
    k = F.normalize(F.linear(x0, W["w_k.weight"]).view(1, -1, H, D), dim=-1)
    v = F.normalize(F.linear(x0, W["w_v.weight"]).view(1, -1, H, D), dim=-1)
    dl = 0.1 * torch.sigmoid(F.linear(x0, W["w_delta.weight"]))
    o64, p64 = sssd_closed.sssd_scan_closed_c(q.numpy(), k.numpy(), v.numpy(), dl.numpy())
    o_norm = F.rms_norm(torch.from_numpy(o64).float(), (D,), W["head_rmsnorm.weight"])
    y_ref = F.linear(o_norm.reshape(1, -1, H * D), W["w_out.weight"])
    ey = _rel(ys[0:1].float().cpu(), y_ref)
    ep = _rel(psi[0:1].cpu(), p64)
    nrm = psi.double().reshape(psi.shape[0], H, -1).norm(dim=-1).cpu().numpy()
    en = float(np.abs(nrm / np.sqrt(D) - 1).max())
    print(f"  SSSD item 0: rel y={ey:.2e} state={ep:.2e}; state norm drift (all items) {en:.2e}",
          flush=True)
    assert ey <= 2e-2 and ep <= 2e-2 and en <= 1e-4

    # ---- CHAM sub-layer, item 0, first 64 tokens
    c = layer.cham_memory
    xc, (yc, _) = cap["cham"]
    Wc = {n: p.detach().float().cpu() for n, p in c.state_dict().items()}
    x0 = xc[0:1, :64].float().cpu()
    qc = F.normalize(F.linear(x0, Wc["w_q.weight"]), dim=-1)
    kc = F.normalize(F.linear(x0, Wc["w_k.weight"]), dim=-1)
    vc = F.normalize(F.silu(F.linear(x0, Wc["w_v.weight"])), dim=-1)
    gc = 0.1 * torch.sigmoid(F.linear(x0, Wc["w_gamma.weight"])).squeeze(-1)
    rec, _ = cham_scan.cham_scan_closed(qc.numpy(), kc.numpy(), vc.numpy(), gc.numpy())
    yc_ref = F.rms_norm(F.linear(torch.from_numpy(rec).float(), Wc["w_out.weight"]),
                        (cfg.hidden_dim,), Wc["norm.weight"], eps=c.norm.eps)
    eyc = _rel(yc[0:1, :64].float().cpu(), yc_ref)
    hn = torch.sqrt(hr.double().pow(2).sum((-2, -1)) + hi.double().pow(2).sum((-2, -1))).cpu().numpy()
    ehn = float(np.abs(hn / np.sqrt(cfg.chams_holographic_dim) - 1).max())
    print(f"  CHAM item 0, 64 tokens: rel y={eyc:.2e}; hologram norm drift (all items) {ehn:.2e}",
          flush=True)
    assert eyc <= 2e-2 and ehn <= 1e-4
