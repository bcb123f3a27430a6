"""TEST INFRASTRUCTURE -- fp64 token-sequential closed form of the SSSD scan.

Restates the recurrence of ``verace_v1/modules/sssd_attention.py:160-175``
(R_t = solve(I + X_t, I - X_t), Psi_t = R_t Psi_{t-1}, o_t = Psi_t q_t) one token at a
time, applying R_t in closed form:

    R = I + c(-X + X^2),  c = 2 / (1 + m^2),  m^2 = (delta/2)^2 (|k|^2 |v|^2 - (k.v)^2)

``cayley_closed`` builds R explicitly (pinned against ``torch.linalg.solve`` in the
tests); ``sssd_scan_closed_np`` is the numpy reference; ``sssd_scan_closed_c`` calls
the C build of the same loop (``oracle/sssd_oracle.c``) for sizes numpy cannot
finish quickly.  Never imported by the product.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libsssd_oracle.so")
_lib = None


def cayley_closed(k: np.ndarray, v: np.ndarray, delta: float) -> np.ndarray:
    """Explicit R = (I + X)^-1 (I - X) for X = (delta/2)(k v^T - v k^T), fp64."""
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    D = k.shape[0]
    h = 0.5 * float(delta)
    X = h * (np.outer(k, v) - np.outer(v, k))
    m2 = h * h * max(float(k @ k) * float(v @ v) - float(k @ v) ** 2, 0.0)
    c = 2.0 / (1.0 + m2)
    return np.eye(D) + c * (-X + X @ X)


def sssd_scan_closed_np(q, k, v, delta, psi0: Optional[np.ndarray] = None,
                        return_norms: bool = False):
    """fp64 sequential scan.  q, k, v: [B,T,H,D]; delta: [B,T,H]; psi0: [B,H,D,D] or None.

    Returns (o [B,T,H,D], psi_T [B,H,D,D]) and, if asked, norms [B,H,T] (Frobenius
    norm of Psi_t after each token).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    delta = np.asarray(delta, dtype=np.float64)
    if delta.ndim == 4:
        delta = delta[..., 0]
    B, T, H, D = q.shape
    if psi0 is None:
        psi = np.broadcast_to(np.eye(D), (B, H, D, D)).copy()
    else:
        psi = np.asarray(psi0, dtype=np.float64).copy()
    out = np.zeros((B, T, H, D))
    norms = np.zeros((B, H, T))
    for t in range(T):
        kt, vt, qt = k[:, t], v[:, t], q[:, t]          # [B,H,D]
        h = 0.5 * delta[:, t]                            # [B,H]
        kk = np.einsum("bhd,bhd->bh", kt, kt)
        vv = np.einsum("bhd,bhd->bh", vt, vt)
        kv = np.einsum("bhd,bhd->bh", kt, vt)
        c = 2.0 / (1.0 + h * h * np.maximum(kk * vv - kv * kv, 0.0))
        a = np.einsum("bhi,bhij->bhj", kt, psi)
        b = np.einsum("bhi,bhij->bhj", vt, psi)
        h_ = h[..., None]
        c_ = c[..., None]
        alpha = c_ * (-h_ * b + h_ * h_ * (kv[..., None] * b - vv[..., None] * a))
        beta = c_ * (h_ * a + h_ * h_ * (kv[..., None] * a - kk[..., None] * b))
        psi = psi + kt[..., :, None] * alpha[..., None, :] + vt[..., :, None] * beta[..., None, :]
        out[:, t] = np.einsum("bhij,bhj->bhi", psi, qt)
        norms[:, :, t] = np.sqrt(np.einsum("bhij,bhij->bh", psi, psi))
    if return_norms:
        return out, psi, norms
    return out, psi


def build_c_oracle() -> str:
    """Compile ``oracle/sssd_oracle.c`` (make) if the shared library is missing or stale."""
    src = os.path.join(_HERE, "sssd_oracle.c")
    if (not os.path.exists(_LIB_PATH)) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        build_c_oracle()
        lib = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.c_void_p
        lib.oracle_sssd_scan_f64.argtypes = [fp, fp, fp, fp, fp, fp, fp, fp,
                                             ctypes.c_long, ctypes.c_long, ctypes.c_long,
                                             ctypes.c_long, ctypes.c_int]
        lib.oracle_sssd_scan_f64.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def sssd_scan_closed_c(q, k, v, delta, psi0=None, want_out: bool = True,
                       want_norms: bool = False, threads: Optional[int] = None):
    """Same as :func:`sssd_scan_closed_np`, computed by the C oracle (OpenMP over B*H).

    Inputs are converted to float32 arrays (exact for bf16/fp16 data); psi0 to float64.
    Returns (o or None, psi_T[, norms]).
    """
    lib = _load()
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    delta = np.ascontiguousarray(delta, dtype=np.float32)
    if delta.ndim == 4:
        delta = np.ascontiguousarray(delta[..., 0])
    B, T, H, D = q.shape
    p0 = None if psi0 is None else np.ascontiguousarray(psi0, dtype=np.float64)
    out = np.zeros((B, T, H, D)) if want_out else None
    psi = np.zeros((B, H, D, D))
    norms = np.zeros((B, H, T)) if want_norms else None
    nt = threads or len(os.sched_getaffinity(0))
    rc = lib.oracle_sssd_scan_f64(_ptr(q), _ptr(k), _ptr(v), _ptr(delta), _ptr(p0), _ptr(out),
                                  _ptr(psi), _ptr(norms), B, T, H, D, nt)
    if rc != 0:
        raise RuntimeError(f"oracle_sssd_scan_f64 returned {rc}")
    if want_norms:
        return out, psi, norms
    return out, psi


def scan_closed(q, k, v, delta, psi0=None) -> Tuple[np.ndarray, np.ndarray]:
    """Convenience: C oracle when it builds, else numpy (identical arithmetic order aside)."""
    try:
        return sssd_scan_closed_c(q, k, v, delta, psi0)
    except (OSError, subprocess.CalledProcessError):
        return sssd_scan_closed_np(q, k, v, delta, psi0)


def identity_substitute(k, v, delta):
    """The reference's non-finite guard as an input substitution (``sssd_attention.py:45-71``):
    a token-head whose Cayley factor is not finite (a NaN/Inf in its k, v or delta) gets
    R = I, which is what the closed form yields for k = v = 0, delta = 0.  Returns cleaned
    float64 copies of k [B,T,H,D], v and delta [B,T,H] and the bad mask [B,T,H].
    Pinned against the eager restatement of the guard (``sssd_eager.solve_cayley``) in
    tests/test_oracle_pins.py."""
    k = np.array(k, dtype=np.float64)
    v = np.array(v, dtype=np.float64)
    delta = np.array(delta, dtype=np.float64)
    if delta.ndim == 4:
        delta = delta[..., 0]
    with np.errstate(over="ignore", invalid="ignore"):
        kk = (k * k).sum(-1)
        vv = (v * v).sum(-1)
    bad = ~(np.isfinite(kk) & np.isfinite(vv) & np.isfinite(delta))
    k[bad] = 0.0
    v[bad] = 0.0
    delta[bad] = 0.0
    return k, v, delta, bad
