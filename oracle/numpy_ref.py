"""NumPy sequential-recurrence restatement of the three recurrent operators.

TEST INFRASTRUCTURE ONLY.  This module is the oracle: it is imported by
``tests/``, by ``__graft_entry__.smoke()`` (as the checker) and by the
``cpu_baseline`` leg of ``bench.py`` (as the timed CPU path).  The product
library never imports, links or calls anything under ``oracle/``.

Each function restates the arithmetic of one reference CUDA kernel in the
reference's operation order, as a Python loop over the sequence axis that is
vectorised over every independent axis.  ``dtype=np.float64`` is the accuracy
yardstick; ``dtype=np.float32`` keeps every intermediate in fp32 and is the
"reference CPU path" that the benchmark times.

Parity pins (closed forms, invariants, brute force, special cases) live in
``tests/test_oracle_pins.py``; the header of each function names what pins it.
"""

from __future__ import annotations

import numpy as np

# Constants exactly as the reference spells them (single-precision literals).
LOG2E_F32 = np.float32(1.4426950408889634)        # M_LOG2E cast to float (selective_scan_fwd_kernel.cuh:172)
PI_F32 = np.float32(3.14159265358979323846)       # kPi (mamba3_siso_fwd.cu:15)
TWO_PI_F32 = np.float32(2.0) * PI_F32             # kTwoPi (mamba3_siso_fwd.cu:16)
L2NORM_EPS_F32 = np.float32(1.0e-6)               # kL2NormEps (gated_deltanet2_fwd.cu:14)


def _as(x, dtype):
    return None if x is None else np.asarray(x).astype(dtype, copy=False)


def _present(x) -> bool:
    """Optional inputs are zero-element tensors (ort_common.h:93-95)."""
    return x is not None and np.asarray(x).size > 0


# ---------------------------------------------------------------------------
# SelectiveScanFn
# ---------------------------------------------------------------------------

def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                   delta_softplus=False, dtype=np.float64, return_state=False):
    """Output 0 of SelectiveScanFn.

    Follows selective_scan_fwd_kernel.cuh:114-127 (D, delta_bias), :150-163
    (bias, softplus with the x<=20 branch, delta*u, D*u), :166-270 (per-state
    exp2 discretisation, affine scan, C contraction), :272-281 (output stored
    before the z gate) and selective_scan_fn_ort.cpp:77-117 (group-dim insertion
    for rank-3 B/C, variable-vs-constant B/C by rank, n_groups taken from B).
    ``z`` is accepted and ignored: output 0 never depends on it
    (selective_scan_fwd_kernel.cuh:280 vs :296-299).

    Shapes: u, delta [Bt,D,L]; A [D,N]; B, C [D,N] or [Bt,N,L] or [Bt,G,N,L];
    D, delta_bias [D] or absent.  Returns y [Bt,D,L] in ``dtype``; with
    ``return_state`` returns ``(y, h)``, h [Bt,D,N] the scan state after the
    last token (the Mamba selective_scan_fn's last_state; zeros when L = 0).
    """
    u = _as(u, dtype); delta = _as(delta, dtype)
    A = _as(A, dtype); B = _as(B, dtype); C = _as(C, dtype)
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    if B.ndim == 3:
        B = B[:, None]
    if C.ndim == 3:
        C = C[:, None]
    b_var = B.ndim >= 3
    c_var = C.ndim >= 3
    ngroups = B.shape[1] if b_var else 1
    ratio = dim // ngroups
    group_of_d = np.arange(dim) // ratio                     # [D]
    Dv = _as(D, dtype) if _present(D) else np.zeros(dim, dtype)
    bias = _as(delta_bias, dtype) if _present(delta_bias) else np.zeros(dim, dtype)

    dlt = delta + bias[None, :, None]
    if delta_softplus:
        with np.errstate(over="ignore"):
            sp = np.log1p(np.exp(dlt))
        dlt = np.where(dlt <= dtype(20.0), sp, dlt).astype(dtype, copy=False)
    du = dlt * u
    out = Dv[None, :, None] * u
    log2e = dtype(LOG2E_F32) if dtype == np.float32 else np.float64(np.log2(np.e))
    if dtype == np.float32:
        A2 = (A * LOG2E_F32).astype(np.float32)             # A_val *= kLog2e in fp32
    else:
        A2 = A * log2e

    # Per-(b,d,n) coefficient tensors used inside the scan.
    if b_var:
        Bsel = B[:, group_of_d]                              # [Bt,D,N,L]
    if c_var:
        Csel = C[:, group_of_d] if b_var else C[:, np.zeros(dim, np.int64)]
    if not b_var and not c_var:
        bc_const = B * C                                     # BC_val folded (kernel.cuh:205-210)

    h = np.zeros((batch, dim, dstate), dtype)
    for t in range(seqlen):
        a = np.exp2(dlt[:, :, t, None] * A2[None])           # exp2f(delta * A * log2e)
        if b_var:
            bterm = Bsel[:, :, :, t] * du[:, :, t, None]
        else:
            bterm = np.broadcast_to(du[:, :, t, None], h.shape)
        h = a * h + bterm                                    # SSMScanOp: (a1*a0, a1*b0 + b1)
        if c_var:
            cval = Csel[:, :, :, t] if b_var else B[None] * Csel[:, :, :, t]
        elif b_var:
            cval = C[None]
        else:
            cval = bc_const[None]
        # out_vals += thread_data.y * C_val, accumulated over n in order 0..N-1
        acc = out[:, :, t].copy()
        for n in range(dstate):
            acc = acc + h[:, :, n] * cval[..., n]
        out[:, :, t] = acc
    return (out, h) if return_state else out


# ---------------------------------------------------------------------------
# GatedDeltaNet2Fn
# ---------------------------------------------------------------------------

def gdn2_prepare(q, k, g, beta, scale, use_qk_l2norm, dtype=np.float64):
    """Per (b,t,h) row: normalised q (times scale), normalised k, exp(g), beta*k.

    Follows gated_deltanet2_fwd.cu:39-76 (prepare kernel): q_mul = scale *
    rsqrt(sum q^2 + 1e-6), k_mul = rsqrt(sum k^2 + 1e-6) when the L2 norm is on,
    else q_mul = scale and k_mul = 1.
    """
    q = _as(q, dtype); k = _as(k, dtype); g = _as(g, dtype); beta = _as(beta, dtype)
    eps = dtype(L2NORM_EPS_F32)
    sc = dtype(np.float32(scale))   # the scale attribute is a float (gated_deltanet2_fn_ort.cpp:47)
    if use_qk_l2norm:
        q_mul = sc * (dtype(1.0) / np.sqrt((q * q).sum(-1, keepdims=True) + eps))
        k_mul = dtype(1.0) / np.sqrt((k * k).sum(-1, keepdims=True) + eps)
    else:
        q_mul = np.full(q.shape[:-1] + (1,), sc, dtype)
        k_mul = np.ones(k.shape[:-1] + (1,), dtype)
    qn = (q * q_mul).astype(dtype, copy=False)
    kn = (k * k_mul).astype(dtype, copy=False)
    dec = np.exp(g).astype(dtype, copy=False)
    bk = (beta * kn).astype(dtype, copy=False)
    return qn, kn, dec, bk


def gated_deltanet2(q, k, v, g, beta, w, initial_state=None, scale=1.0,
                    use_qk_l2norm=True, dtype=np.float64, return_state=False):
    """Output of GatedDeltaNet2Fn.

    Recurrence of gated_deltanet2_fwd.cu:82-140 (register path) and :142-233
    (generic path), identical math: per token, S[i,:] *= exp(g_i); erase_j =
    sum_i beta_i khat_i S[i,j]; write_j = w_j v_j - erase_j; S[i,j] += khat_i
    write_j; o_j = sum_i qhat_i S[i,j].  Shapes: q, k, g, beta [B,T,H,K];
    v, w [B,T,H,V]; initial_state [B,H,K,V] or absent.  Returns [B,T,H,V];
    with ``return_state`` returns ``(o, S)``, S [B,H,K,V] the state after the
    last token.
    """
    qn, kn, dec, bk = gdn2_prepare(q, k, g, beta, scale, use_qk_l2norm, dtype)
    v = _as(v, dtype); w = _as(w, dtype)
    batch, seqlen, nheads, dk = qn.shape
    dv = v.shape[-1]
    if _present(initial_state):
        S = _as(initial_state, dtype).copy()
    else:
        S = np.zeros((batch, nheads, dk, dv), dtype)
    out = np.empty((batch, seqlen, nheads, dv), dtype)
    for t in range(seqlen):
        S *= dec[:, t, :, :, None]
        erase = np.einsum("bhk,bhkv->bhv", bk[:, t], S)
        write = w[:, t] * v[:, t] - erase
        S += kn[:, t, :, :, None] * write[:, :, None, :]
        out[:, t] = np.einsum("bhk,bhkv->bhv", qn[:, t], S)
    return (out, S) if return_state else out


# ---------------------------------------------------------------------------
# Mamba3SisoFn
# ---------------------------------------------------------------------------

def _wrap_two_pi(x, dtype):
    """wrap_two_pi (mamba3_siso_fwd.cu:26-28): x - 2pi * floor(x / 2pi)."""
    tp = dtype(TWO_PI_F32)
    return x - tp * np.floor(x / tp)


def _sigmoid(x, dtype):
    return dtype(1.0) / (dtype(1.0) + np.exp(-x))


def mamba3_siso(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D=None, Z=None,
                dtype=np.float64, input_states=None, return_state=False):
    """Output of Mamba3SisoFn (forward, no input/final state, no cu_seqlens).

    Follows mamba3_siso_fwd.cu:79-171: per step the angle state is advanced by
    tanh(angle) * dt * pi and wrapped to [0, 2pi) (:82-86); q = Q + Q_bias and
    k = K + K_bias, qk is the *unrotated* dot product (:89-106); pairs p < A
    are rotated by the angle state (:108-123); gamma = dt * sigmoid(trap) and
    the trapezoid look-ahead dt[t+1] * (1 - sigmoid(trap[t+1])) (:126-134);
    the state decays by exp(adt) before the readout (:140-143); y = q_rot . S
    + (D + qk * gamma) * V, gated by silu(Z) when present (:146-161); then
    S += V (x) k_rot * (gamma + look-ahead) (:164-169).

    Shapes: Q, K [B,T,Hq,N]; V [B,T,H,P]; ADT, DT, Trap [B,H,T]; Q_bias,
    K_bias [H,N]; Angles [B,T,H,A]; D [H] or absent; Z [B,T,H,P] or absent.

    States (a widening; the reference rejects them, mamba3_siso_fn_ort.cpp:50-55):
    ``input_states`` = (ssm [B,H,P,N], angle [B,H,A], k [B,H,N], v [B,H,P]) starts
    from S = ssm + v (x) k * DT_0 (1 - sigmoid(Trap_0)) (the previous call's last
    token's look-ahead, :126-134) and theta = angle; ``return_state`` also
    returns those four after the last token (its rotated k and its V).
    """
    Q = _as(Q, dtype); K = _as(K, dtype); V = _as(V, dtype)
    ADT = _as(ADT, dtype); DT = _as(DT, dtype); Trap = _as(Trap, dtype)
    Qb = _as(Q_bias, dtype); Kb = _as(K_bias, dtype); Ang = _as(Angles, dtype)
    batch, seqlen, nheads_qk, n = Q.shape
    nheads, p_dim = V.shape[2], V.shape[3]
    a_dim = Ang.shape[3]
    grp = nheads // nheads_qk
    gidx = np.arange(nheads) // grp
    has_d = _present(D)
    has_z = _present(Z)
    Dv = _as(D, dtype) if has_d else np.zeros(nheads, dtype)
    Zv = _as(Z, dtype) if has_z else None
    pi = dtype(PI_F32)

    out = np.empty((batch, seqlen, nheads, p_dim), dtype)
    sig_trap = _sigmoid(Trap, dtype)                          # [B,H,T]
    if input_states is not None:
        s_in, a_in, k_in, v_in = (_as(x, dtype) for x in input_states)
        look0 = DT[:, :, 0] * (dtype(1.0) - sig_trap[:, :, 0])   # [B,H]
        S = s_in + v_in[..., :, None] * (k_in[..., None, :] * look0[..., None, None])
        theta = a_in.copy()
    else:
        S = np.zeros((batch, nheads, p_dim, n), dtype)
        theta = np.zeros((batch, nheads, a_dim), dtype)
    k_rot = np.zeros((batch, nheads, n), dtype)
    for t in range(seqlen):
        dt = DT[:, :, t]                                       # [B,H]
        theta = _wrap_two_pi(theta + np.tanh(Ang[:, t]) * dt[..., None] * pi, dtype)
        q = Q[:, t][:, gidx] + Qb[None]                        # [B,H,N]
        k = K[:, t][:, gidx] + Kb[None]
        qk = (q * k).sum(-1)                                   # [B,H]
        phi = np.zeros((batch, nheads, n // 2), dtype)
        phi[..., :a_dim] = theta
        c = np.cos(phi); s = np.sin(phi)
        q0, q1 = q[..., 0::2], q[..., 1::2]
        k0, k1 = k[..., 0::2], k[..., 1::2]
        q_rot = np.empty_like(q); k_rot = np.empty_like(k)
        q_rot[..., 0::2] = q0 * c - q1 * s
        q_rot[..., 1::2] = q0 * s + q1 * c
        k_rot[..., 0::2] = k0 * c - k1 * s
        k_rot[..., 1::2] = k0 * s + k1 * c
        gamma = dt * sig_trap[:, :, t]
        if t + 1 < seqlen:
            shifted = DT[:, :, t + 1] * (dtype(1.0) - sig_trap[:, :, t + 1])
        else:
            shifted = np.zeros_like(gamma)
        k_scaled = k_rot * (gamma + shifted)[..., None]
        S *= np.exp(ADT[:, :, t])[..., None, None]
        y = np.einsum("bhn,bhpn->bhp", q_rot, S) + (Dv[None] + qk * gamma)[..., None] * V[:, t]
        if has_z:
            zt = Zv[:, t]
            y = y * (zt * _sigmoid(zt, dtype))
        out[:, t] = y
        S += V[:, t][..., None] * k_scaled[:, :, None, :]
    if return_state:
        return out, (S, theta, k_rot, V[:, seqlen - 1].copy())
    return out


# ---------------------------------------------------------------------------
# SoftmaxCPU (CPU-EP op in the same domain)
# ---------------------------------------------------------------------------

def softmax_cpu(x, axis=-1):
    """softmax_cpu_ort.cpp:20-114: max-subtract, exp, normalise; inv_sum = 0 when
    the sum is 0 (:75).  fp32 throughout, sum accumulated in axis order."""
    x = np.asarray(x, np.float32)
    ax = axis + x.ndim if axis < 0 else axis
    xm = np.moveaxis(x, ax, -1)
    mx = xm.max(-1, keepdims=True)
    e = np.exp(xm - mx).astype(np.float32)
    s = np.zeros(e.shape[:-1] + (1,), np.float32)
    for i in range(e.shape[-1]):
        s = s + e[..., i:i + 1]
    inv = np.where(s > 0, np.float32(1.0) / np.where(s > 0, s, 1), np.float32(0.0)).astype(np.float32)
    return np.moveaxis(e * inv, -1, ax)
