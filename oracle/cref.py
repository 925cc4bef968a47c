"""ctypes front end of the C restatement (``oracle/xm_oracle.c``).

TEST INFRASTRUCTURE ONLY (the oracle): imported by ``tests/``, the smoke check
and the benchmark's ``cpu_baseline`` leg.  The product never imports it.

Functions take NumPy arrays with the operator's own input layout (the same
arguments as ``oracle.numpy_ref``) and return the output in fp64 (``dtype=
np.float64``) or fp32 (``dtype=np.float32``).  The shared object is built by
``make -C oracle``; :func:`build` runs that.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libxm_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)


def build(force: bool = False) -> str:
    """Compile the C restatement with gcc (make -C oracle)."""
    if force and os.path.exists(_LIB_PATH):
        os.remove(_LIB_PATH)
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _fp(x):
    if x is None:
        return None, None
    a = np.ascontiguousarray(np.asarray(x, np.float32))
    if a.size == 0:
        return None, None
    return a, a.ctypes.data_as(_f32p)


def _out(shape, dtype):
    o = np.empty(shape, dtype)
    ct = ctypes.c_double if dtype == np.float64 else ctypes.c_float
    return o, o.ctypes.data_as(ctypes.POINTER(ct))


def _sfx(dtype):
    if dtype not in (np.float32, np.float64):
        raise ValueError("dtype must be np.float32 or np.float64")
    return "_f64" if dtype == np.float64 else "_f32"


def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                   delta_softplus=False, dtype=np.float64, return_state=False):
    """See xmo_selective_scan in xm_oracle.c.  ``z`` is ignored (dead input).
    With ``return_state`` returns ``(y, last_state)``, last_state [B,D,N]."""
    u_, up = _fp(u); d_, dp = _fp(delta); A_, Ap = _fp(A)
    B_ = np.asarray(B, np.float32); C_ = np.asarray(C, np.float32)
    batch, dim, seqlen = np.shape(u)
    dstate = np.shape(A)[1]
    if B_.ndim == 3:
        B_ = B_[:, None]
    if C_.ndim == 3:
        C_ = C_[:, None]
    b_var = int(B_.ndim >= 3); c_var = int(C_.ndim >= 3)
    gb = B_.shape[1] if b_var else 1
    gc = C_.shape[1] if c_var else 1
    B_, Bp = _fp(B_); C_, Cp = _fp(C_)
    D_, Dp = _fp(D); bi_, bp = _fp(delta_bias)
    out, op = _out((batch, dim, seqlen), dtype)
    st, sp = _out((batch, dim, dstate), dtype) if return_state else (None, None)
    getattr(lib(), "xmo_selective_scan" + _sfx(dtype))(
        up, dp, Ap, Bp, Cp, Dp, bp, batch, dim, seqlen, dstate, b_var, c_var, gb, gc,
        int(bool(delta_softplus)), op, sp)
    return (out, st) if return_state else out


def gated_deltanet2(q, k, v, g, beta, w, initial_state=None, scale=1.0,
                    use_qk_l2norm=True, dtype=np.float64, return_state=False):
    """See xmo_gated_deltanet2 in xm_oracle.c.  With ``return_state`` returns
    ``(o, final_state)``, final_state [B,H,K,V]."""
    q_, qp = _fp(q); k_, kp = _fp(k); v_, vp = _fp(v)
    g_, gp = _fp(g); b_, bp = _fp(beta); w_, wp = _fp(w)
    s_, sp = _fp(initial_state)
    batch, seqlen, nheads, dk = q_.shape
    dv = v_.shape[3]
    out, op = _out((batch, seqlen, nheads, dv), dtype)
    st, stp = _out((batch, nheads, dk, dv), dtype) if return_state else (None, None)
    getattr(lib(), "xmo_gated_deltanet2" + _sfx(dtype))(
        qp, kp, vp, gp, bp, wp, sp, batch, seqlen, nheads, dk, dv,
        ctypes.c_float(float(scale)), int(bool(use_qk_l2norm)), op, stp)
    return (out, st) if return_state else out


def mamba3_siso(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D=None, Z=None,
                dtype=np.float64, input_states=None, return_state=False):
    """See xmo_mamba3_siso in xm_oracle.c.  ``input_states`` is ``(ssm [B,H,P,N],
    angle [B,H,A], k [B,H,N], v [B,H,P])`` or None; with ``return_state``
    returns ``(y, (ssm, angle, k, v))``, the same four after the last token."""
    Q_, Qp = _fp(Q); K_, Kp = _fp(K); V_, Vp = _fp(V)
    a_, ap = _fp(ADT); dt_, dtp = _fp(DT); tr_, trp = _fp(Trap)
    qb_, qbp = _fp(Q_bias); kb_, kbp = _fp(K_bias); an_, anp = _fp(Angles)
    D_, Dp = _fp(D); Z_, Zp = _fp(Z)
    batch, seqlen, nheads_qk, n = Q_.shape
    nheads, p = V_.shape[2], V_.shape[3]
    a_dim = an_.shape[3]
    ins = input_states if input_states is not None else (None, None, None, None)
    (is_, isp), (ia_, iap), (ik_, ikp), (iv_, ivp) = (_fp(x) for x in ins)
    out, op = _out((batch, seqlen, nheads, p), dtype)
    if return_state:
        shapes = ((batch, nheads, p, n), (batch, nheads, a_dim), (batch, nheads, n), (batch, nheads, p))
        fs = [_out(sh, dtype) for sh in shapes]
    else:
        fs = [(None, None)] * 4
    getattr(lib(), "xmo_mamba3_siso" + _sfx(dtype))(
        Qp, Kp, Vp, ap, dtp, trp, qbp, kbp, anp, Dp, Zp, batch, seqlen, nheads, nheads_qk,
        n, p, a_dim, isp, iap, ikp, ivp, op, *(x[1] for x in fs))
    return (out, tuple(x[0] for x in fs)) if return_state else out


def _setup_signatures():
    L = lib()
    for sfx in ("_f32", "_f64"):
        fn = getattr(L, "xmo_selective_scan" + sfx)
        fn.restype = None
        fn = getattr(L, "xmo_gated_deltanet2" + sfx)
        fn.restype = None
        fn = getattr(L, "xmo_mamba3_siso" + sfx)
        fn.restype = None


def softmax_cpu(x, axis=-1, dtype=np.float32):
    """See xmo_softmax_cpu in xm_oracle.c (fp32: the reference's operations and order)."""
    a = np.asarray(x, np.float32, order="C")
    ax = axis + a.ndim if axis < 0 else axis
    if not 0 <= ax < a.ndim:
        raise ValueError("axis out of range")
    outer = int(np.prod(a.shape[:ax], dtype=np.int64))
    inner = int(np.prod(a.shape[ax + 1:], dtype=np.int64))
    o, op = _out(a.shape, dtype)
    if a.size == 0:
        return o
    fn = getattr(lib(), "xmo_softmax_cpu" + _sfx(dtype))
    fn.restype = None
    fn(a.ctypes.data_as(_f32p), ctypes.c_size_t(outer), ctypes.c_size_t(a.shape[ax]), ctypes.c_size_t(inner), op)
    return o
