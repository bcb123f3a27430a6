"""verace_amd -- MI355X (gfx950) SSSD Cayley-scan attention for Verace V1.

Drop-in replacements for the reference's SSSD hot path:

* ``SSSDAttention``            <- ``verace_v1.modules.sssd_attention.SSSDAttention``
* ``launch_sssd_hip_scan``     <- ``verace_v1.serving.triton_kernels.launch_sssd_triton_scan``
* ``SSSDScanFunction`` / ``sssd_scan`` / ``launch_sssd_hip_scan_bwd``
                               -- the scan with its backward (training; the reference
                                  differentiates its eager path instead)
* ``launch_sssd_hip_scan_fused`` -- the scan with the projections' normalisation, delta,
                                  mask and head RMSNorm fused in (on x @ [W_q; W_k; W_v; W_delta].T)
* ``sssd_step_``               -- in-place single-token decode step (opt-in)
* ``sssd_step_fused_``         -- the same step with the projections' normalisation, delta,
                                  mask and head RMSNorm fused in (on one row of the stacked
                                  projection per item)
* ``SSSDStateCache``           -- per-layer decode state pools with copy-on-write
                                  branches (replaces the ``layer_states`` lists of
                                  ``acd_engine.py`` / ``hyper_generate.py``)
* ``newton_schulz_unitary_retraction`` / ``parallel_newton_schulz_retraction``
                               <- ``verace_v1.modules.cham_memory`` (same names)
* ``launch_cham_hip_update``   <- ``verace_v1.serving.triton_kernels.launch_cham_triton_update``
                               (CHAM holographic scan, holographic_dim <= 4096)
* ``cham_step_``               -- in-place single-token CHAM step (opt-in)
* ``cham_step_fused_``         -- the same step with silu, the normalisations and gamma fused in
* ``launch_cham_hip_update_fused`` -- the CHAM scan from the identity with the same fusion
* ``ContinuousHolographicMemory`` <- ``verace_v1.modules.cham_memory.ContinuousHolographicMemory``
* ``ManifoldContinuousMoE`` / ``SiTUGLU`` <- ``verace_v1.modules.mcmoe`` / ``.activations`` (torch ops)
* ``VeraceV1Layer`` / ``VeraceV1Model`` / ``VeraceV1Config`` / ``DecodeState``
                               -- the layer harness (``backbone.py:21-210``, ACDE
                                  ``acd_engine.py:36-167``) with batched in-place decode
* ``HAS_HIP``                  <- ``verace_v1.serving.triton_kernels.HAS_TRITON``

``torch.ops.verace.{sssd_scan, sssd_scan_bwd, sssd_step_, sssd_scan_fused, cham_scan, cham_step_,
ns_retraction}`` are the same launchers registered as torch operators with fake kernels and
autograd (``ops.py``), for FakeTensor / meta tracing and ``torch.compile``.

All compute runs in ``libverace_sssd.so`` (C ABI: ``include/verace_sssd.h``).
"""
from .hip_kernels import (HAS_HIP, SSSDScanFunction, cham_step_, cham_step_fused_,
                          launch_cham_hip_update, launch_cham_hip_update_fused,
                          launch_sssd_hip_scan, launch_sssd_hip_scan_bwd,
                          launch_sssd_hip_scan_fused,
                          newton_schulz_unitary_retraction, parallel_newton_schulz_retraction,
                          sssd_scan, sssd_step_, sssd_step_fused_)
from . import ops  # noqa: F401  (torch.ops.verace.*: the launchers as traceable operators)
from .sssd_attention import SSSDAttention
from .cham_memory import ContinuousHolographicMemory
from .mcmoe import ManifoldContinuousMoE, SiTUGLU
from .backbone import (AdaptiveCognitiveDepthEngine, DecodeGraph, DecodeState, LayerDecodeState,
                       VeraceV1Config, VeraceV1Layer, VeraceV1Model)
from .state_cache import SlotTable, SSSDStateCache

__all__ = [
    "HAS_HIP",
    "SSSDAttention",
    "SSSDScanFunction",
    "sssd_scan",
    "launch_sssd_hip_scan_bwd",
    "SSSDStateCache",
    "SlotTable",
    "launch_sssd_hip_scan",
    "launch_sssd_hip_scan_fused",
    "launch_cham_hip_update",
    "launch_cham_hip_update_fused",
    "sssd_step_",
    "sssd_step_fused_",
    "cham_step_",
    "cham_step_fused_",
    "ContinuousHolographicMemory",
    "ManifoldContinuousMoE",
    "SiTUGLU",
    "AdaptiveCognitiveDepthEngine",
    "DecodeState",
    "DecodeGraph",
    "LayerDecodeState",
    "VeraceV1Config",
    "VeraceV1Layer",
    "VeraceV1Model",
    "newton_schulz_unitary_retraction",
    "parallel_newton_schulz_retraction",
]
