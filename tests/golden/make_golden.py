"""Writes tests/golden/sssd_module_golden.npz from the reference implementation.

Run in the development container only (the reference is not present on the GPU box):

    python tests/golden/make_golden.py [/root/reference]

Why an import is needed: the oracle's math (closed-form Cayley factor, prefix product,
module restatement) is pinned by library routines, brute force and invariants in
tests/test_oracle_pins.py.  What none of those can pin is the *seed-dependent
construction* of ``SSSDAttention`` (which parameters exist, their shapes and the
order in which they draw from the RNG, ``verace_v1/modules/sssd_attention.py:80-101``)
and the exact fp32 rounding of the reference's eager forward.  This script records,
for the reference's own test shapes (``tests/test_triton_kernels.py:88-148``,
``tests/test_sssd.py:10-26``), the parameters the reference creates after
``torch.manual_seed(seed)``, the input ``x`` and the eager forward's output and state.
Only data is written (inputs and outputs); no reference source is copied.

All tensors are created on CPU (the reference tests use CUDA RNG streams, which differ);
the eager path is the one the reference takes on CPU (sssd_attention.py:129 gate).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "sssd_module_golden.npz")


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from verace_v1.modules.sssd_attention import SSSDAttention  # noqa: E402

    cases = []
    # (name, seed, b, s, head_dim, num_heads, hidden, kind)
    for (b, s, D, H) in [(2, 8, 16, 2), (1, 1, 16, 1), (2, 13, 16, 2), (2, 8, 24, 2)]:
        cases.append((f"match_b{b}_s{s}_d{D}_h{H}", 0, b, s, D, H, H * D, "plain"))
    cases.append(("halted_b2_s10_d16_h2", 1, 2, 10, 16, 2, 32, "halted"))
    cases.append(("chain_b2_s6_d16_h2", 2, 2, 6, 16, 2, 32, "chain"))
    cases.append(("norm_b2_s8_d64_h2", 0, 2, 8, 64, 2, 128, "plain"))

    blobs = {}
    names = []
    for name, seed, b, s, D, H, hidden, kind in cases:
        torch.manual_seed(seed)
        model = SSSDAttention(hidden_dim=hidden, num_heads=H, head_dim=D)
        x = torch.randn(b, s, hidden)
        for pname, p in model.state_dict().items():
            blobs[f"{name}/param/{pname}"] = p.detach().numpy().copy()
        blobs[f"{name}/x"] = x.numpy().copy()
        blobs[f"{name}/meta"] = np.array([b, s, D, H, hidden], dtype=np.int64)
        with torch.no_grad():
            if kind == "plain":
                out, st = model(x, return_state=True)
            elif kind == "halted":
                mask = torch.ones(b, s, dtype=torch.bool)
                mask[:, s // 2:] = False
                blobs[f"{name}/active_mask"] = mask.numpy().copy()
                out, st = model(x, return_state=True, active_mask=mask)
            else:  # chain: state of x1 feeds x2
                x2 = torch.randn(b, s, hidden)
                blobs[f"{name}/x2"] = x2.numpy().copy()
                out1, st1 = model(x, return_state=True)
                blobs[f"{name}/out1"] = out1.numpy().copy()
                blobs[f"{name}/state1"] = st1.numpy().copy()
                out, st = model(x2, initial_state=st1, return_state=True)
        blobs[f"{name}/out"] = out.numpy().copy()
        blobs[f"{name}/state"] = st.numpy().copy()
        names.append(name)
    blobs["cases"] = np.array(names)
    np.savez_compressed(OUT, **blobs)
    print(f"wrote {OUT} ({len(names)} cases, torch {torch.__version__})")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
