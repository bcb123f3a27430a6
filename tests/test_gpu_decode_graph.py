"""The decode step captured in a HIP graph (verace_amd.DecodeGraph) against the eager
``decode_step`` it records (the generator's per-token call, hyper_generate.py:58-63).

A small random model (hidden 64, 2 layers, H 2, D 32, CHAM 32 on the step kernel, and CHAM 30,
which takes the general scan + retraction route) is prefilled from fresh states; then the same
token ids are stepped eagerly on one copy of the states and by graph replays on another.  The
replays run with the program's own eager work and synchronisations between them, and every
replay's logits and the states after it are compared with the eager step's.  Bar: fp32 max
abs difference <= 1e-5 (the same kernels run in both; the graph only removes the host launch
cost).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _copy(st):
    from verace_amd import DecodeState, LayerDecodeState
    return DecodeState([LayerDecodeState(
        l.sssd.clone(), (l.cham[0].clone(), l.cham[1].clone()),
        None if l.cham_readout is None else (l.cham_readout[0].clone(), l.cham_readout[1].clone()))
        for l in st.layers])


@pytest.mark.parametrize("cham_dim,static_depth", [(32, False), (32, True), (30, False)])
def test_decode_graph_matches_eager(device, cham_dim, static_depth):
    from verace_amd import DecodeGraph, VeraceV1Config, VeraceV1Model
    print(f"[case] DecodeGraph cham_dim={cham_dim} static_depth={static_depth}", flush=True)
    torch.manual_seed(3)
    cfg = VeraceV1Config(vocab_size=300, hidden_dim=64, num_layers=2, num_heads=2, head_dim=32,
                         chams_holographic_dim=cham_dim, mcmoe_rank=4, mcmoe_num_components=16,
                         energy_halting_threshold=0.0474)
    m = VeraceV1Model(cfg).to(device).eval()
    B = 3
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 300, (B, 12), generator=g).to(device)
    nxt = torch.randint(0, 300, (4, B, 1), generator=g).to(device)
    with torch.no_grad():
        _, st = m.prefill(ids, static_depth=static_depth)
        st_e, st_g = _copy(st), _copy(st)
        graph = DecodeGraph(m, st_g, B, static_depth=static_depth)
        # construction does not advance the states it was given
        for a, b in zip(st_g.layers, st.layers):
            assert torch.equal(a.sssd, b.sssd) and torch.equal(a.cham[0], b.cham[0])
        for i in range(nxt.shape[0]):
            ref = m.decode_step(nxt[i], st_e, static_depth=static_depth)
            torch.cuda.synchronize()
            got = graph.step(nxt[i]).clone()
            torch.cuda.synchronize()
            e = float((got - ref).abs().max())
            es = max(float((a.sssd - b.sssd).abs().max()) for a, b in zip(st_g.layers, st_e.layers))
            eh = max(max(float((a.cham[j] - b.cham[j]).abs().max()) for j in (0, 1))
                     for a, b in zip(st_g.layers, st_e.layers))
            print(f"  replay {i}: logits {e:.2e} sssd {es:.2e} cham {eh:.2e}", flush=True)
            assert e <= 1e-5 and es <= 1e-5 and eh <= 1e-5
