"""Fixed-depth and ACDE layer harness around the accelerated SSSD and CHAM scans.

``VeraceV1Layer`` restates ``verace_v1/modules/backbone.py:21-101`` (same sub-module names,
order and residual structure: block-residual mix, ``sssd_norm`` -> SSSD, ``cham_norm`` ->
CHAM, ``mcmoe_norm`` -> M-CMoE), with ``SSSDAttention`` and ``ContinuousHolographicMemory``
running on the HIP kernels and the M-CMoE as torch ops.  ``VeraceV1Model`` restates the
text path of ``backbone.py:104-210`` (embedding tied to ``lm_head``, the layers, ACDE or the
static loop, final norm); the vision encoder and the energy critic are not built (images are
out of scope; ``vision_encoder.*`` / ``energy_critic.*`` keys are ignored when loading a
reference ``state_dict``), but ``from_seed`` reproduces the reference's seeded weights when it
is given the torch RNG state the reference has right after building its vision encoder.

``AdaptiveCognitiveDepthEngine`` restates ``acd_engine.py:13-167``.  The reference runs the
layers per batch item on the gathered active tokens ([1, S_active, d]) and threads a
``(sssd_state, cham_hologram)`` per layer and item.  Here every layer runs once on the whole
batch with the active tokens as ``active_mask``: an inactive token has delta = gamma = 0,
i.e. R = I and U = I exactly, so each item's states and its active tokens' outputs are
those of the gathered sequence; outputs of inactive tokens are discarded as in the
reference.  (The block residual the reference threads through ACDE never holds a snapshot:
its per-item buffers start as [s, 0, d] and the assignment at acd_engine.py:123 broadcasts
into zero columns, so no layer mixes; the harness keeps that.)

Decode (``prefill`` / ``decode_step``): the model's states live in a :class:`DecodeState`
of batched tensors per layer (SSSD ``[B, H, D, D]``, CHAM ``(H_real, H_imag) [B, h, h]`` and,
when the CHAM state is not unitary, its readout state ``NS_3(H)``), updated in place by the
single-token step kernels: one SSSD launch and one CHAM launch per layer for the whole
batch, where the reference's generator re-runs the forward per item at seq_len 1
(``hyper_generate.py:58-63``).  ``to_layer_states`` / ``from_layer_states`` convert to and
from the reference's per-layer, per-item lists.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
import torch.nn as nn

from .cham_memory import ContinuousHolographicMemory
from .hip_kernels import newton_schulz_unitary_retraction
from .mcmoe import ManifoldContinuousMoE
from .sssd_attention import SSSDAttention


@dataclass
class VeraceV1Config:
    """The fields of ``verace_v1/config.py:15-73`` the text model uses (same defaults)."""
    vocab_size: int = 163840
    hidden_dim: int = 1024
    num_layers: int = 12
    num_heads: int = 8
    head_dim: int = 128
    spectral_dim: int = 256
    chams_holographic_dim: int = 1024
    mcmoe_rank: int = 32
    mcmoe_num_components: int = 64
    max_cognitive_depth: int = 12
    min_cognitive_depth: int = 2
    energy_halting_threshold: float = 0.99
    rms_norm_eps: float = 1e-6


class VeraceV1Layer(nn.Module):
    def __init__(self, layer_idx: int, config: VeraceV1Config):
        super().__init__()
        self.layer_idx = layer_idx
        self.config = config
        self.sssd_norm = nn.RMSNorm(config.hidden_dim, eps=config.rms_norm_eps)
        self.sssd_attn = SSSDAttention(hidden_dim=config.hidden_dim, num_heads=config.num_heads,
                                       head_dim=config.head_dim, spectral_dim=config.spectral_dim)
        self.cham_norm = nn.RMSNorm(config.hidden_dim, eps=config.rms_norm_eps)
        self.cham_memory = ContinuousHolographicMemory(hidden_dim=config.hidden_dim,
                                                       holographic_dim=config.chams_holographic_dim)
        self.mcmoe_norm = nn.RMSNorm(config.hidden_dim, eps=config.rms_norm_eps)
        self.mcmoe = ManifoldContinuousMoE(hidden_dim=config.hidden_dim, rank=config.mcmoe_rank,
                                           num_components=config.mcmoe_num_components,
                                           beta1=4.0, beta2=25.0)

    def forward(self, h_in: torch.Tensor, block_residual: Optional[torch.Tensor] = None,
                sssd_state: Optional[torch.Tensor] = None,
                cham_hologram: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                active_mask: Optional[torch.Tensor] = None):
        """backbone.py:53-101: returns (h_out, block_residual, sssd_state, cham_hologram)."""
        b, s, h = h_in.shape
        flat_h = h_in.reshape(b * s, h)
        if block_residual is None:
            block_residual = flat_h.new_zeros(b * s, 0, h)
        if block_residual.shape[1] > 0:  # AttnRes mixing over the committed snapshots
            w = torch.softmax(torch.matmul(flat_h.unsqueeze(1), block_residual.transpose(-1, -2)).squeeze(1), dim=-1)
            h_in = (flat_h + torch.matmul(w.unsqueeze(1), block_residual).squeeze(1)).view(b, s, h)
        if self.layer_idx % 12 == 0:
            block_residual = torch.cat([block_residual, flat_h.unsqueeze(1)], dim=1)
        sssd_out, new_sssd_state = self.sssd_attn(self.sssd_norm(h_in), initial_state=sssd_state,
                                                  return_state=True, active_mask=active_mask)
        h_mid1 = h_in + sssd_out
        cham_out, new_holo = self.cham_memory(self.cham_norm(h_mid1), initial_hologram=cham_hologram,
                                              active_mask=active_mask)
        h_mid2 = h_mid1 + cham_out
        h_out = h_mid2 + self.mcmoe(self.mcmoe_norm(h_mid2))
        return h_out, block_residual, new_sssd_state, new_holo

    def step_(self, h_in: torch.Tensor, st: "LayerDecodeState",
              active_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One token per item (h_in [B, 1, hidden]) with this layer's states updated in
        place; the same sub-layers as :meth:`forward` (no block residual: a decode call's
        layers never receive a snapshot, see the module docstring)."""
        h_mid1 = h_in + self.sssd_attn.step_(self.sssd_norm(h_in), st.sssd, active_mask)
        cham_out = self.cham_memory.step_(self.cham_norm(h_mid1), st.cham, st.cham_readout, active_mask)
        h_mid2 = h_mid1 + cham_out
        return h_mid2 + self.mcmoe(self.mcmoe_norm(h_mid2))


class AdaptiveCognitiveDepthEngine(nn.Module):
    """acd_engine.py:13-34 (the halting unit, same init)."""

    def __init__(self, hidden_dim: int = 16384, energy_threshold: float = 0.99):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.energy_threshold = energy_threshold
        self.w_halting = nn.Linear(hidden_dim, 1)
        nn.init.constant_(self.w_halting.bias, -3.0)
        nn.init.normal_(self.w_halting.weight, std=0.01)

    def compute_halting_probability(self, h_l: torch.Tensor) -> torch.Tensor:
        return torch.sigmoid(self.w_halting(h_l)).squeeze(-1)

    def run(self, layers, h_in: torch.Tensor, max_depth: int, min_depth: int,
            initial_layer_states=None, step_states: Optional["DecodeState"] = None,
            static_control: bool = False):
        """acd_engine.py:36-167 on the whole batch (see the module docstring).  With
        ``step_states`` (T = 1) the layers take their in-place step instead of the forward.
        ``static_control`` takes no decision from device values (every layer runs, always with
        the active mask; the results are the same), so the loop can be captured in a HIP graph.
        Returns (final_h, depth_counts, layer_states as per-layer lists of per-item tuples,
        or None with step_states)."""
        b, s, d = h_in.shape
        h_curr = h_in.clone()
        final_h = torch.zeros_like(h_in)
        acc = torch.zeros(b, s, device=h_in.device, dtype=h_in.dtype)
        depth = torch.zeros(b, s, device=h_in.device, dtype=h_in.dtype)
        active = torch.ones(b, s, device=h_in.device, dtype=torch.bool)
        n_layers = min(len(layers), max_depth)
        states_out = None
        if step_states is None:
            states_out = [(list(initial_layer_states[l]) if initial_layer_states is not None
                           and l < len(initial_layer_states) and initial_layer_states[l] is not None
                           else [None] * b) for l in range(n_layers)]
        for l_idx in range(n_layers):
            if not static_control and not bool(active.any()):
                break
            layer = layers[l_idx]
            item_on = active.any(dim=1)                              # items with work here
            mask = active if static_control or not bool(active.all()) else None
            if step_states is not None:
                out = layer.step_(h_curr, step_states.layers[l_idx], mask)
            else:
                sst, holo = _stack_states(states_out[l_idx], item_on, layer, h_in)
                out, _, new_s, new_h = layer(h_curr, sssd_state=sst, cham_hologram=holo, active_mask=mask)
                for i in range(b):
                    if bool(item_on[i]):
                        states_out[l_idx][i] = (new_s[i:i + 1], (new_h[0][i:i + 1], new_h[1][i:i + 1]))
            h_next = torch.where(active.unsqueeze(-1), out, h_curr)
            p = self.compute_halting_probability(h_next)
            if l_idx < min_depth:
                p = torch.zeros_like(p)
            new_acc = acc + p
            halted = (new_acc >= self.energy_threshold) & active
            still = active & ~halted
            rem = (1.0 - acc).clamp(min=0.0)
            w = torch.where(halted, rem, p)
            upd = active | halted
            final_h = final_h + (w * upd.to(h_in.dtype)).unsqueeze(-1) * h_next
            depth = depth + active.to(h_in.dtype)
            depth = depth + rem * halted.to(h_in.dtype)
            acc = new_acc
            active = still
            h_curr = h_next
        if static_control or bool(active.any()):
            rem = (1.0 - acc).clamp(min=0.0)
            final_h = final_h + (rem * active.to(h_in.dtype)).unsqueeze(-1) * h_curr
            depth = depth + rem * active.to(h_in.dtype)
        return final_h, depth, states_out


def _stack_states(per_item, item_on, layer, like):
    """Batched (sssd_state, hologram) for a layer from per-item tuples; None when no item
    has a state yet.  Items without a state start from the identity (the reference's None)."""
    if all(s is None for s in per_item):
        return None, None
    b = len(per_item)
    a = layer.sssd_attn
    hd = layer.cham_memory.holographic_dim
    dev = like.device
    eyeD = torch.eye(a.head_dim, device=dev).expand(a.num_heads, -1, -1)
    eyeh = torch.eye(hd, device=dev)
    sst = torch.stack([s[0][0].float() if s is not None else eyeD for s in per_item])
    hr = torch.stack([s[1][0][0].float() if s is not None else eyeh for s in per_item])
    hi = torch.stack([s[1][1][0].float() if s is not None else torch.zeros_like(eyeh) for s in per_item])
    return sst.contiguous(), (hr.contiguous(), hi.contiguous())


@dataclass
class LayerDecodeState:
    sssd: torch.Tensor                                   # [B, H, D, D] float32
    cham: Tuple[torch.Tensor, torch.Tensor]              # raw (H_real, H_imag) [B, h, h]
    cham_readout: Optional[Tuple[torch.Tensor, torch.Tensor]] = None  # NS_3(H) if H not unitary


@dataclass
class DecodeState:
    """Per-layer batched decode states (updated in place by ``decode_step``)."""
    layers: List[LayerDecodeState]

    def to_layer_states(self):
        """The reference's ``layer_states[l][i] = (sssd_state, (H_real, H_imag))`` (copies)."""
        out = []
        for st in self.layers:
            b = st.sssd.shape[0]
            out.append([(st.sssd[i:i + 1].clone(), (st.cham[0][i:i + 1].clone(), st.cham[1][i:i + 1].clone()))
                        for i in range(b)])
        return out

    @staticmethod
    def from_layer_states(layer_states, model: "VeraceV1Model", batch: int, device) -> "DecodeState":
        """From the reference's per-layer, per-item lists (None = identity).  The CHAM readout
        state is NS_3(H) of each hologram (computed once here), so later steps need no
        retraction."""
        layers = []
        for l, layer in enumerate(model.layers):
            per_item = layer_states[l] if layer_states is not None and l < len(layer_states) else [None] * batch
            like = torch.empty(0, device=device)
            sst, holo = _stack_states(per_item, torch.ones(batch, dtype=torch.bool), layer, like)
            if sst is None:
                layers.append(model._fresh_layer_state(layer, batch, device))
                continue
            rr, ri = newton_schulz_unitary_retraction(holo[0], holo[1], 3)
            layers.append(LayerDecodeState(sst, holo, (rr.contiguous(), ri.contiguous())))
        return DecodeState(layers)


class VeraceV1Model(nn.Module):
    def __init__(self, config: VeraceV1Config, rng_state_after_vision: Optional[torch.Tensor] = None):
        """Same construction order as backbone.py:110-142.  The reference builds its vision
        encoder between ``lm_head`` and the layers; with ``rng_state_after_vision`` (the torch
        CPU RNG state the reference has at that point) the RNG is set to it instead, so the
        seeded weights of every built parameter equal the reference's."""
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_dim)
        self.lm_head = nn.Linear(config.hidden_dim, config.vocab_size, bias=False)
        self.embed_tokens.weight = self.lm_head.weight  # weight tying (backbone.py:116)
        if rng_state_after_vision is not None:
            torch.set_rng_state(rng_state_after_vision)
        self.layers = nn.ModuleList([VeraceV1Layer(i, config) for i in range(config.num_layers)])
        self.acd_engine = AdaptiveCognitiveDepthEngine(config.hidden_dim, config.energy_halting_threshold)
        self.final_norm = nn.RMSNorm(config.hidden_dim, eps=config.rms_norm_eps)

    def load_reference_state_dict(self, sd: dict, strict: bool = True):
        """A reference ``VeraceV1Model.state_dict()``; the vision encoder's and the energy
        critic's entries (not built here) are skipped."""
        sd = {k: v for k, v in sd.items()
              if not k.startswith("vision_encoder.") and not k.startswith("energy_critic.")}
        return self.load_state_dict(sd, strict=strict)

    def forward(self, input_ids: torch.Tensor, images=None, use_adaptive_depth: bool = True,
                return_hidden: bool = False, layer_states: Optional[List] = None,
                return_layer_states: bool = False):
        """backbone.py:144-210 (text path): (logits, depth_counts[, hidden][, layer_states])."""
        if images is not None:
            raise NotImplementedError("verace_amd.VeraceV1Model: the vision path is not built")
        b, s = input_ids.shape
        x = self.embed_tokens(input_ids)
        states = None
        if use_adaptive_depth:
            final_h, depth, states = self.acd_engine.run(
                self.layers, x, self.config.max_cognitive_depth, self.config.min_cognitive_depth,
                initial_layer_states=layer_states)
        else:
            h = x
            for layer in self.layers:
                h, _, _, _ = layer(h)
            final_h = h
            depth = torch.full((b, s), float(len(self.layers)), device=input_ids.device, dtype=x.dtype)
        norm_h = self.final_norm(final_h)
        logits = self.lm_head(norm_h)
        if return_hidden and return_layer_states:
            return logits, depth, norm_h, states
        if return_hidden:
            return logits, depth, norm_h
        if return_layer_states:
            return logits, depth, states
        return logits, depth

    # ---------------------------------------------------------------- decode
    def _fresh_layer_state(self, layer, batch, device) -> LayerDecodeState:
        a = layer.sssd_attn
        hd = layer.cham_memory.holographic_dim
        sssd = torch.eye(a.head_dim, device=device).expand(batch, a.num_heads, -1, -1).contiguous()
        hr = torch.eye(hd, device=device).expand(batch, -1, -1).contiguous()
        return LayerDecodeState(sssd, (hr, torch.zeros_like(hr)), None)

    def prefill(self, input_ids: torch.Tensor, static_depth: bool = False):
        """Prompt pass from fresh states: (logits, DecodeState).  From the identity start every
        CHAM state is unitary, so its readout state is H itself (no retraction)."""
        b, s = input_ids.shape
        x = self.embed_tokens(input_ids)
        st = DecodeState([])
        if static_depth:
            h = x
            for layer in self.layers:
                h, _, sssd, holo = layer(h)
                st.layers.append(LayerDecodeState(sssd, holo, None))
            final_h = h
        else:
            final_h, _, per = self.acd_engine.run(self.layers, x, self.config.max_cognitive_depth,
                                                  self.config.min_cognitive_depth)
            for l, layer in enumerate(self.layers):
                if l < len(per) and any(t is not None for t in per[l]):
                    sst, holo = _stack_states(per[l], None, layer, x)
                    st.layers.append(LayerDecodeState(sst, holo, None))
                else:
                    st.layers.append(self._fresh_layer_state(layer, b, x.device))
        return self.lm_head(self.final_norm(final_h)), st

    def decode_step(self, next_ids: torch.Tensor, state: DecodeState, static_depth: bool = False,
                    static_control: bool = False):
        """One token per item (next_ids [B, 1]); the states are updated in place.  The same
        function as ``forward(next_ids, layer_states=...)`` (ACDE) or the static loop."""
        x = self.embed_tokens(next_ids)
        if static_depth:
            h = x
            for l, layer in enumerate(self.layers):
                h = layer.step_(h, state.layers[l])
            final_h = h
        else:
            final_h, _, _ = self.acd_engine.run(self.layers, x, self.config.max_cognitive_depth,
                                                self.config.min_cognitive_depth, step_states=state,
                                                static_control=static_control)
        return self.lm_head(self.final_norm(final_h))


class DecodeGraph:
    """``decode_step`` captured once in a HIP graph (torch.cuda.CUDAGraph) and replayed per
    token: the ~40 small launches per layer of a batch-64 decode step (projections, norms,
    M-CMoE, halting) are otherwise bound by host launch cost.  The graph reads the next token
    ids from :attr:`ids` and writes the logits into :attr:`logits`; the states of ``state`` are
    updated in place by every replay.  Warm-up runs (needed before capture) use a copy of the
    states, so ``state`` is not advanced by the construction."""

    def __init__(self, model: VeraceV1Model, state: DecodeState, batch: int,
                 static_depth: bool = False, warmup: int = 2):
        dev = state.layers[0].sssd.device
        self.ids = torch.zeros(batch, 1, dtype=torch.long, device=dev)
        scratch = DecodeState([LayerDecodeState(
            l.sssd.clone(), (l.cham[0].clone(), l.cham[1].clone()),
            None if l.cham_readout is None else (l.cham_readout[0].clone(), l.cham_readout[1].clone()))
            for l in state.layers])
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                model.decode_step(self.ids, scratch, static_depth, static_control=True)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        del scratch
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = model.decode_step(self.ids, state, static_depth, static_control=True)

    def step(self, next_ids: torch.Tensor) -> torch.Tensor:
        """Advance every item by one token; returns the logits [B, 1, vocab] (the graph's
        output buffer, overwritten by the next step)."""
        self.ids.copy_(next_ids)
        self.graph.replay()
        return self.logits
