"""The layer's third sub-block, M-CMoE, as torch ops (not on the accelerated path; the layer
harness needs it to run the reference's layer).

``SiTUGLU`` restates ``verace_v1/modules/activations.py:8-31`` and
``ManifoldContinuousMoE`` restates ``verace_v1/modules/mcmoe.py:20-120`` with the same
parameter names and creation order (so seeded construction and ``state_dict`` loading
match the reference).  The sparse top-K sum
``sum_k w_k U_{j_k} (sigma_{j_k} * (V_{j_k} x))`` (the reference's loop at :101-117, which
gathers a [tokens, hidden, rank] basis copy per k) is evaluated as two dense GEMMs over all
components with the non-selected components' coefficients set to zero: the same sum, with
no per-token gathers.
"""
from __future__ import annotations

import torch
import torch.nn as nn


class SiTUGLU(nn.Module):
    """``[b1 tanh(W_g x / b1) sigmoid(W_g x)] * [b2 tanh(W_u x / b2)]`` (activations.py:8-31)."""

    def __init__(self, in_features: int, hidden_features: int, beta1: float = 4.0,
                 beta2: float = 25.0):
        super().__init__()
        self.in_features = in_features
        self.hidden_features = hidden_features
        self.beta1 = beta1
        self.beta2 = beta2
        self.w_gate = nn.Linear(in_features, hidden_features, bias=False)
        self.w_up = nn.Linear(in_features, hidden_features, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        g = self.w_gate(x)
        u = self.w_up(x)
        return (self.beta1 * torch.tanh(g / self.beta1) * torch.sigmoid(g)) * \
            (self.beta2 * torch.tanh(u / self.beta2))


class ManifoldContinuousMoE(nn.Module):
    def __init__(self, hidden_dim: int = 16384, rank: int = 32, num_components: int = 64,
                 top_k_components: int = 8, beta1: float = 4.0, beta2: float = 25.0):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.rank = rank
        self.num_components = num_components
        self.top_k_components = top_k_components
        self.base_situ_glu = SiTUGLU(hidden_dim, hidden_dim * 2, beta1=beta1, beta2=beta2)
        self.base_w_down = nn.Linear(hidden_dim * 2, hidden_dim, bias=False)
        self.u_basis = nn.Parameter(torch.randn(num_components, hidden_dim, rank) * 0.02)
        self.v_basis = nn.Parameter(torch.randn(num_components, rank, hidden_dim) * 0.02)
        self.router = nn.Linear(hidden_dim, num_components, bias=False)
        self.hyper_sigma = nn.Linear(hidden_dim, num_components * rank, bias=False)
        self.norm = nn.RMSNorm(hidden_dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, s, d = x.shape
        C, r = self.num_components, self.rank
        xf = x.reshape(b * s, d)
        base_out = self.base_w_down(self.base_situ_glu(xf))
        # keep-top-k before the softmax (mcmoe.py:82-87)
        kv = min(self.top_k_components, C)
        logits = self.router(xf)
        top_l, top_i = torch.topk(logits, k=kv, dim=-1)
        masked = torch.full_like(logits, float("-inf")).scatter(-1, top_i, top_l)
        weights = torch.softmax(masked, dim=-1)                   # exactly 0 off the top k
        sigma = torch.sigmoid(self.hyper_sigma(xf)).view(b * s, C, r)
        # v_proj[n, j, :] = V_j x_n for every component, then the selected ones' coefficients
        vproj = (xf @ self.v_basis.reshape(C * r, d).t()).view(b * s, C, r)
        coef = (vproj * sigma * weights.unsqueeze(-1)).reshape(b * s, C * r)
        adapt = coef @ self.u_basis.permute(0, 2, 1).reshape(C * r, d)
        return (base_out + self.norm(adapt)).view(b, s, d)
