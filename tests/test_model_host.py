"""The layer harness on the host (no GPU): the seeded construction of the CPU config's model
(VeraceV1Model seed 0, hidden 256, 2 layers, H 4, D 64, vocab 32000, CHAM 1024) reproduces the
reference's parameters bit for bit, given the torch RNG state the reference has right after
building its vision encoder (tests/golden/model_golden.npz, written by
tests/golden/make_golden_model.py from the reference itself); and the tiny model's reference
state_dict loads into the harness with every key accounted for.
"""
import os

import numpy as np
import pytest
import torch

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "model_golden.npz")


def _golden():
    if not os.path.exists(GOLDEN):
        pytest.skip("model golden fixture not generated")
    return np.load(GOLDEN, allow_pickle=False)


def cpu_config_model():
    from verace_amd import VeraceV1Config, VeraceV1Model
    z = _golden()
    cfg = VeraceV1Config(vocab_size=32000, hidden_dim=256, num_layers=2, num_heads=4, head_dim=64)
    torch.manual_seed(0)
    rng = torch.from_numpy(z["cpu/rng_after_vision"].copy())
    return VeraceV1Model(cfg, rng_state_after_vision=rng), z


def tiny_model():
    from verace_amd import VeraceV1Config, VeraceV1Model
    z = _golden()
    V, Hd, L, H, D, h, r, C = (int(x) for x in z["tiny/config"])
    cfg = VeraceV1Config(vocab_size=V, hidden_dim=Hd, num_layers=L, num_heads=H, head_dim=D,
                         chams_holographic_dim=h, mcmoe_rank=r, mcmoe_num_components=C,
                         energy_halting_threshold=float(z["tiny/halting_threshold"]))
    m = VeraceV1Model(cfg)
    sd = {k[len("tiny/param/"):]: torch.from_numpy(z[k].copy()) for k in z.files if k.startswith("tiny/param/")}
    missing, unexpected = m.load_reference_state_dict(sd, strict=False)
    return m, z, missing, unexpected


def test_cpu_config_seeded_weights_equal_reference():
    m, z = cpu_config_model()
    names = [str(n) for n in z["cpu/param_names"]]
    ours = dict(m.named_parameters())
    skipped = [n for n in names if n.startswith("energy_critic.")]
    for n in names:
        if n in skipped:
            continue
        assert n in ours, n
        p = ours[n].detach().double().reshape(-1)
        d = z[f"cpu/digest/{n}"]
        head = p[:8].numpy()
        assert np.array_equal(head, d[2:2 + head.size]), n  # leading values bit-exact
        assert abs(float(p.sum()) - d[0]) <= 1e-9 * max(1.0, abs(d[0])), n
        assert abs(float((p * p).sum()) - d[1]) <= 1e-9 * max(1.0, abs(d[1])), n
    # every parameter the harness builds is one of the reference's
    assert set(ours) <= set(names)


def test_tiny_reference_state_dict_loads():
    m, z, missing, unexpected = tiny_model()
    assert not missing and not unexpected
