"""Decode state cache: per-layer pools of SSSD states with copy-on-write branches.

The reference threads decode state as Python lists, ``layer_states[l][i] =
(sssd_state, cham_hologram)`` (``acd_engine.py:85-126``), runs the batch one item at a
time, and branches tree search by shallow-copying those lists so that every candidate
token starts from the same cached state and returns a fresh one
(``hyper_generate.py:97-121``; ``sssd_attention.py:103-182`` never mutates
``initial_state``).  Here the states of every layer live in one device tensor
``[L, N, H, D, D]`` fp32 (N slots per layer), and a *sequence handle* names one
sequence (a batch item or a tree-search branch):

* ``new`` makes handles that start from the identity (no slot until first written);
* ``fork`` makes handles that share their parent's slot on every layer (no copy);
* ``step`` runs one batched decode step of a layer for a list of handles with one
  kernel launch.  A handle that is the only holder of its slot is updated in place; a
  handle whose slot is shared reads the shared slot and writes a fresh one, so the copy
  of copy-on-write is the step's own write, never an extra pass;
* ``write`` / ``read`` move whole states in and out (prefill results, export);
* ``release`` returns a handle's slots once no other handle holds them.

The bookkeeping and the launches are native (``vmi_state_cache_*`` in
``libverace_sssd.so``; the slot of every item travels in the kernel arguments, so a
step costs one C call and one launch).  :class:`SlotTable` is the bookkeeping alone
(no device needed); :class:`SSSDStateCache` adds the device pool.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib

_I64P = ctypes.POINTER(ctypes.c_int64)
_I32P = ctypes.POINTER(ctypes.c_int)


def _handles(handles) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(handles, dtype=np.int64).reshape(-1))


def _check(status: int, what: str) -> None:
    if status == 1:
        raise ValueError(f"verace_amd: {what}: invalid argument (unknown, released or repeated "
                         "handle, or layer out of range)")
    if status == 6:
        raise RuntimeError(f"verace_amd: {what}: state cache layer full")
    _lib.check(status, what)


class SlotTable:
    """Slot assignment and reference counts of ``num_layers`` pools of ``num_slots`` slots
    (the native cache object, without a device pool unless ``pool_ptr`` is given)."""

    def __init__(self, num_layers: int, num_slots: int, num_heads: int = 1, head_dim: int = 1,
                 pool_ptr: Optional[int] = None):
        self._lib = _lib.load()
        self.num_layers = num_layers
        self.num_slots = num_slots
        self._h = ctypes.c_void_p()
        _check(self._lib.vmi_state_cache_create(num_layers, num_slots, num_heads, head_dim,
                                                pool_ptr, ctypes.byref(self._h)),
               "vmi_state_cache_create")

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.vmi_state_cache_destroy(h)
            self._h = None

    # -- handles ------------------------------------------------------------------
    def new(self, n: int = 1) -> List[int]:
        out = np.empty(n, dtype=np.int64)
        _check(self._lib.vmi_state_cache_new(self._h, n, out.ctypes.data_as(_I64P)),
               "vmi_state_cache_new")
        return out.tolist()

    def fork(self, parent: int, n: int = 1) -> List[int]:
        out = np.empty(n, dtype=np.int64)
        _check(self._lib.vmi_state_cache_fork(self._h, int(parent), n, out.ctypes.data_as(_I64P)),
               "vmi_state_cache_fork")
        return out.tolist()

    def release(self, handles: Sequence[int]) -> None:
        hs = _handles(handles)
        _check(self._lib.vmi_state_cache_release(self._h, hs.ctypes.data_as(_I64P), len(hs)),
               "vmi_state_cache_release")

    # -- queries and planning ----------------------------------------------------
    def slots(self, layer: int, handles: Sequence[int]) -> np.ndarray:
        hs = _handles(handles)
        out = np.empty(len(hs), dtype=np.int32)
        _check(self._lib.vmi_state_cache_slots(self._h, layer, hs.ctypes.data_as(_I64P), len(hs),
                                               out.ctypes.data_as(_I32P)), "vmi_state_cache_slots")
        return out

    def phys(self, handle: int) -> np.ndarray:
        """Slot of ``handle`` at every layer (-1: still the identity)."""
        return np.array([self.slots(l, [handle])[0] for l in range(self.num_layers)])

    @property
    def refs(self) -> np.ndarray:
        out = np.empty((self.num_layers, self.num_slots), dtype=np.int32)
        for l in range(self.num_layers):
            _check(self._lib.vmi_state_cache_refs(self._h, l, out[l].ctypes.data_as(_I32P), None),
                   "vmi_state_cache_refs")
        return out

    def free_slots(self, layer: int) -> int:
        n = ctypes.c_int64(0)
        _check(self._lib.vmi_state_cache_refs(self._h, layer, None, ctypes.byref(n)),
               "vmi_state_cache_refs")
        return n.value

    def plan_step(self, layer: int, handles: Sequence[int]) -> Tuple[np.ndarray, np.ndarray]:
        """Slots read (-1: identity) and written by one step of ``layer`` over ``handles``,
        with the table updated as if the step had run (no launch)."""
        hs = _handles(handles)
        src = np.empty(len(hs), dtype=np.int32)
        dst = np.empty(len(hs), dtype=np.int32)
        _check(self._lib.vmi_state_cache_plan(self._h, layer, hs.ctypes.data_as(_I64P), len(hs),
                                              src.ctypes.data_as(_I32P), dst.ctypes.data_as(_I32P)),
               "vmi_state_cache_plan")
        return src, dst

    def plan_write(self, layer: int, handles: Sequence[int]) -> np.ndarray:
        """Slots to which whole new states of ``handles`` are written (copy-on-write as
        for a step, without reading the old state)."""
        return self.plan_step(layer, handles)[1]


class SSSDStateCache:
    """``[num_layers, num_slots, H, D, D]`` fp32 states on one device, addressed by handles.

    With ``hologram_dim`` the cache also holds each handle's CHAM hologram (the second half
    of the reference's ``(sssd_state, cham_hologram)`` tuple) in ``holograms``
    ``[num_layers, num_slots, 2, h, h]`` (real plane, imaginary plane) under the same slot as
    its SSSD state: :meth:`cham_step` steps them in place after :meth:`step` of the same layer
    and handles.  Cached holograms are taken to have started from the identity (unitary, so
    their Newton-Schulz readout is the hologram itself).

    All launches go to the current stream of ``device``; the steps of one cache must stay
    on one stream.  D = 128 runs the persistent decode-step kernel, other D up to 256 the
    token-sequential kernel.
    """

    def __init__(self, num_layers: int, num_slots: int, num_heads: int, head_dim: int,
                 device: Optional[torch.device] = None, hologram_dim: Optional[int] = None):
        device = torch.device(device if device is not None else "cuda")
        if device.type != "cuda":
            raise RuntimeError("verace_amd: the state cache lives on a HIP device")
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.device = device
        self.states = torch.zeros(num_layers, num_slots, num_heads, head_dim, head_dim,
                                  dtype=torch.float32, device=device)
        self.table = SlotTable(num_layers, num_slots, num_heads, head_dim,
                               self.states.data_ptr())
        self.hologram_dim = hologram_dim
        self.holograms = None
        if hologram_dim is not None:
            self.holograms = torch.zeros(num_layers, num_slots, 2, hologram_dim, hologram_dim,
                                         dtype=torch.float32, device=device)
            _check(self.table._lib.vmi_state_cache_attach_hologram(
                self.table._h, hologram_dim, ctypes.c_void_p(self.holograms.data_ptr())),
                "vmi_state_cache_attach_hologram")

    # -- handles (host only) -------------------------------------------------------
    def new(self, n: int = 1) -> List[int]:
        return self.table.new(n)

    def fork(self, parent: int, n: int = 1) -> List[int]:
        return self.table.fork(parent, n)

    def release(self, handles: Sequence[int]) -> None:
        self.table.release(handles)

    # -- device work ---------------------------------------------------------------
    def step(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             delta: torch.Tensor, handles) -> torch.Tensor:
        """One decode step of ``layer`` for ``handles`` (item b of q/k/v/delta continues
        handles[b]; a prebuilt int64 numpy array avoids a conversion per call).
        q, k, v: [B, 1, H, D] or [B, H, D]; delta: [B, 1, H] or [B, H].
        Returns o [B, 1, H, D] in q's dtype."""
        H, D = self.num_heads, self.head_dim
        hs = handles if isinstance(handles, np.ndarray) and handles.dtype == np.int64 \
            else _handles(handles)
        B = len(hs)
        q_c = q.reshape(B, 1, H, D).contiguous()
        k_c = k.reshape(B, 1, H, D).to(q.dtype).contiguous()
        v_c = v.reshape(B, 1, H, D).to(q.dtype).contiguous()
        d_c = delta.reshape(B, 1, H).contiguous()
        for name, t in (("q", q_c), ("k", k_c), ("v", v_c), ("delta", d_c)):
            if t.device != self.device:
                raise RuntimeError(f"verace_amd: {name} must be on {self.device}, got {t.device}")
        out = torch.empty_like(q_c)
        P = ctypes.c_void_p
        _check(self.table._lib.vmi_state_cache_step(
            self.table._h, layer, hs.ctypes.data_as(_I64P), B, P(q_c.data_ptr()),
            P(k_c.data_ptr()), P(v_c.data_ptr()), P(d_c.data_ptr()), _lib.dtype_code(q_c.dtype),
            _lib.dtype_code(d_c.dtype), P(out.data_ptr()), _lib.stream_handle(self.device)),
            "vmi_state_cache_step")
        return out

    def cham_step(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  gamma: torch.Tensor, handles) -> torch.Tensor:
        """The in-place CHAM decode step of ``layer`` for the same ``handles`` (same order) as
        the preceding :meth:`step` of that layer: each hologram moves with its SSSD state's
        slot (copy-on-write included).  Once per step: a second call, or one after a fork, a
        release or another plan of the layer, raises ValueError.
        q, k, v: [B, 1, h] or [B, h]; gamma: [B] or [B, 1].
        Returns Re(NS_3(H') q) [B, 1, h] in q's dtype."""
        if self.holograms is None:
            raise RuntimeError("verace_amd: this cache holds no holograms (hologram_dim=None)")
        h = self.hologram_dim
        hs = handles if isinstance(handles, np.ndarray) and handles.dtype == np.int64 \
            else _handles(handles)
        B = len(hs)
        q_c = q.reshape(B, 1, h).contiguous()
        k_c = k.reshape(B, 1, h).to(q.dtype).contiguous()
        v_c = v.reshape(B, 1, h).to(q.dtype).contiguous()
        g_c = gamma.reshape(B).contiguous()
        out = torch.empty_like(q_c)
        lib = self.table._lib
        ws_bytes = ctypes.c_size_t(0)
        _check(lib.vmi_state_cache_cham_workspace_bytes(B, h, ctypes.byref(ws_bytes)),
               "vmi_state_cache_cham_workspace_bytes")
        ws = torch.empty(max(ws_bytes.value, 1), device=self.device, dtype=torch.uint8)
        P = ctypes.c_void_p
        _check(lib.vmi_state_cache_cham_step(
            self.table._h, layer, hs.ctypes.data_as(_I64P), B, P(q_c.data_ptr()), P(k_c.data_ptr()),
            P(v_c.data_ptr()), P(g_c.data_ptr()), _lib.dtype_code(q_c.dtype),
            _lib.dtype_code(g_c.dtype), P(out.data_ptr()), P(ws.data_ptr()), ws_bytes.value,
            _lib.stream_handle(self.device)), "vmi_state_cache_cham_step")
        return out

    def write(self, layer: int, handles: Sequence[int], states: torch.Tensor,
              holograms: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
        """Store whole states [B, H, D, D] (e.g. the final states of a prefill scan) and, for
        a cache with holograms, the raw holograms (H_real, H_imag) [B, h, h] (identity where
        not given)."""
        dst = self.table.plan_write(layer, handles)
        if len(dst):
            idx = torch.from_numpy(dst.astype(np.int64)).to(self.device)
            self.states[layer].index_copy_(0, idx, states.to(torch.float32).reshape(
                len(dst), self.num_heads, self.head_dim, self.head_dim))
            if self.holograms is not None:
                h = self.hologram_dim
                if holograms is None:
                    hr = torch.eye(h, device=self.device).expand(len(dst), h, h)
                    hi = torch.zeros(len(dst), h, h, device=self.device)
                else:
                    hr, hi = holograms
                pair = torch.stack([hr.to(torch.float32).reshape(len(dst), h, h),
                                    hi.to(torch.float32).reshape(len(dst), h, h)], 1)
                self.holograms[layer].index_copy_(0, idx, pair)

    def read_holograms(self, layer: int, handles: Sequence[int]):
        """(H_real, H_imag) [B, h, h] of ``handles`` at ``layer`` (identity where never written)."""
        if self.holograms is None:
            raise RuntimeError("verace_amd: this cache holds no holograms (hologram_dim=None)")
        slots = self.table.slots(layer, handles).astype(np.int64)
        h = self.hologram_dim
        hr = torch.eye(h, dtype=torch.float32, device=self.device).expand(len(slots), h, h).contiguous()
        hi = torch.zeros(len(slots), h, h, dtype=torch.float32, device=self.device)
        have = np.nonzero(slots >= 0)[0]
        if len(have):
            src = torch.from_numpy(slots[have]).to(self.device)
            dst = torch.from_numpy(have).to(self.device)
            sel = self.holograms[layer].index_select(0, src)
            hr[dst] = sel[:, 0]
            hi[dst] = sel[:, 1]
        return hr, hi

    def read(self, layer: int, handles: Sequence[int]) -> torch.Tensor:
        """States [B, H, D, D] of ``handles`` at ``layer`` (identity where never written)."""
        slots = self.table.slots(layer, handles).astype(np.int64)
        H, D = self.num_heads, self.head_dim
        out = torch.eye(D, dtype=torch.float32, device=self.device).expand(
            len(slots), H, D, D).contiguous()
        have = np.nonzero(slots >= 0)[0]
        if len(have):
            src = torch.from_numpy(slots[have]).to(self.device)
            out[torch.from_numpy(have).to(self.device)] = self.states[layer].index_select(0, src)
        return out
