"""Seeded synthetic workloads for the three operators, and their byte counts.

Inputs are drawn with ``np.random.default_rng(seed)`` in fp64, in the fixed
order listed in each generator, and cast to fp32.  The same arrays feed the
device path and the CPU oracle.

Algorithmic bytes = every input byte the output depends on, read once, plus
the output written once.  They exclude scratch, re-reads and SelectiveScan's
``z`` (output 0 does not depend on it):

* SelectiveScanFn:  4 * (3*B*D*L + 2*B*G*N*L + D*N + 2*D)      (u, delta, y; B, C; A; D, bias)
* GatedDeltaNet2Fn: 4 * (4*B*T*H*K + 3*B*T*H*V + [S0] B*H*K*V)  (q, k, g, beta; v, w, o; S0)
* Mamba3SisoFn:     4 * (2*B*T*Hq*N + 2*B*T*H*P + [Z] B*T*H*P + B*T*H*A + 3*B*H*T + 2*H*N + [D] H)
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np


def _softplus(x):
    return np.logaddexp(0.0, x)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


# ---------------------------------------------------------------------------
# SelectiveScanFn
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class SelectiveScanShape:
    batch: int
    dim: int
    seqlen: int
    dstate: int
    groups: int = 1            # G for variable B/C of rank 4; 1 => rank 3
    b_var: bool = True
    c_var: bool = True
    has_d: bool = True
    has_z: bool = True
    has_bias: bool = True
    delta_softplus: bool = True


def selective_scan_inputs(s: SelectiveScanShape, seed: int = 0) -> Dict[str, Optional[np.ndarray]]:
    """Draw order: u, delta, z, delta_bias, A, B, C, D.

    u, delta, z ~ N(0,1) [B,D,L]; delta_bias ~ U(-4,-2) [D];
    A = -exp(U(0, ln 16)) [D,N]; B, C ~ N(0,1) [B,N,L] (or [B,G,N,L] when
    groups > 1, or [D,N] when constant); D ~ N(0,1) [D].
    """
    rng = np.random.default_rng(seed)
    f = np.float32
    shp = (s.batch, s.dim, s.seqlen)
    u = rng.standard_normal(shp).astype(f)
    delta = rng.standard_normal(shp).astype(f)
    z = rng.standard_normal(shp).astype(f) if s.has_z else None
    bias = rng.uniform(-4.0, -2.0, s.dim).astype(f) if s.has_bias else None
    A = (-np.exp(rng.uniform(0.0, np.log(16.0), (s.dim, s.dstate)))).astype(f)

    def bc(var):
        if not var:
            return rng.standard_normal((s.dim, s.dstate)).astype(f)
        if s.groups == 1:
            return rng.standard_normal((s.batch, s.dstate, s.seqlen)).astype(f)
        return rng.standard_normal((s.batch, s.groups, s.dstate, s.seqlen)).astype(f)

    B = bc(s.b_var)
    C = bc(s.c_var)
    D = rng.standard_normal(s.dim).astype(f) if s.has_d else None
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=bias)


def selective_scan_bytes(s: SelectiveScanShape) -> int:
    bcl = 2 * s.batch * s.groups * s.dstate * s.seqlen
    bc = (bcl // 2 if s.b_var else s.dim * s.dstate) + (bcl // 2 if s.c_var else s.dim * s.dstate)
    return 4 * (3 * s.batch * s.dim * s.seqlen + bc + s.dim * s.dstate
                + (s.dim if s.has_d else 0) + (s.dim if s.has_bias else 0))


# ---------------------------------------------------------------------------
# GatedDeltaNet2Fn
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class GatedDeltaNet2Shape:
    batch: int
    seqlen: int
    nheads: int
    dk: int
    dv: int
    initial_state: bool = True
    per_key_gates: bool = False     # False: g, beta drawn per (b,t,h) and broadcast over keys
    l2norm: bool = True

    @property
    def scale(self) -> float:
        return float(1.0 / np.sqrt(self.dk))


def gated_deltanet2_inputs(s: GatedDeltaNet2Shape, seed: int = 0) -> Dict[str, Optional[np.ndarray]]:
    """Draw order: q, k, v, g_raw, beta_raw, w_raw, initial_state.

    q, k, v ~ N(0,1); g = -softplus(N(0,1)); beta = sigmoid(N(0,1)), drawn per
    (b,t,h) and broadcast over keys into the schema's [B,T,H,K] (or per key
    when ``per_key_gates``); w = sigmoid(N(0,1)) [B,T,H,V];
    initial_state ~ N(0, 0.05^2) [B,H,K,V].
    """
    rng = np.random.default_rng(seed)
    f = np.float32
    qk_shape = (s.batch, s.seqlen, s.nheads, s.dk)
    v_shape = (s.batch, s.seqlen, s.nheads, s.dv)
    q = rng.standard_normal(qk_shape).astype(f)
    k = rng.standard_normal(qk_shape).astype(f)
    v = rng.standard_normal(v_shape).astype(f)
    gshape = qk_shape if s.per_key_gates else qk_shape[:3] + (1,)
    g = (-_softplus(rng.standard_normal(gshape))).astype(f)
    beta = _sigmoid(rng.standard_normal(gshape)).astype(f)
    g = np.ascontiguousarray(np.broadcast_to(g, qk_shape))
    beta = np.ascontiguousarray(np.broadcast_to(beta, qk_shape))
    w = _sigmoid(rng.standard_normal(v_shape)).astype(f)
    s0 = (0.05 * rng.standard_normal((s.batch, s.nheads, s.dk, s.dv))).astype(f) if s.initial_state else None
    return dict(q=q, k=k, v=v, g=g, beta=beta, w=w, initial_state=s0)


def gated_deltanet2_bytes(s: GatedDeltaNet2Shape) -> int:
    btH = s.batch * s.seqlen * s.nheads
    return 4 * (4 * btH * s.dk + 3 * btH * s.dv + (s.batch * s.nheads * s.dk * s.dv if s.initial_state else 0))


# ---------------------------------------------------------------------------
# Mamba3SisoFn
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class Mamba3SisoShape:
    batch: int
    seqlen: int
    nheads: int
    headdim: int            # P
    dstate: int             # N
    nheads_qk: int = 0      # 0 => nheads
    angles: int = 0         # 0 => dstate // 2
    has_d: bool = True
    has_z: bool = False

    @property
    def hq(self) -> int:
        return self.nheads_qk or self.nheads

    @property
    def a(self) -> int:
        return self.angles or self.dstate // 2


def mamba3_siso_inputs(s: Mamba3SisoShape, seed: int = 0) -> Dict[str, Optional[np.ndarray]]:
    """Draw order: V, dt_bias, dt_raw, A_log, Q, K, Trap, Angles, D, Q_bias, K_bias, Z.

    V ~ N(0,1) [B,T,H,P]; DT = softplus(N(0,1) + dt_bias[h]), dt_bias ~
    U(-4,-2) [H]; A_h = -exp(U(0, ln 16)); ADT = A_h * DT [B,H,T];
    Q, K ~ N(0,1)/sqrt(N) [B,T,Hq,N]; Trap ~ U(0,1) [B,H,T];
    Angles ~ U(0,1) [B,T,H,A]; D ~ N(0,1) [H]; Q_bias, K_bias ~ N(0,1)/sqrt(N)
    [H,N]; Z ~ N(0,1) [B,T,H,P] when present.
    """
    rng = np.random.default_rng(seed)
    f = np.float32
    B, T, H, P, N = s.batch, s.seqlen, s.nheads, s.headdim, s.dstate
    V = rng.standard_normal((B, T, H, P)).astype(f)
    dt_bias = rng.uniform(-4.0, -2.0, H)
    DT = _softplus(rng.standard_normal((B, H, T)) + dt_bias[None, :, None])
    A = -np.exp(rng.uniform(0.0, np.log(16.0), H))
    ADT = (A[None, :, None] * DT).astype(f)
    DT = DT.astype(f)
    rs = 1.0 / np.sqrt(N)
    Q = (rng.standard_normal((B, T, s.hq, N)) * rs).astype(f)
    K = (rng.standard_normal((B, T, s.hq, N)) * rs).astype(f)
    Trap = rng.uniform(0.0, 1.0, (B, H, T)).astype(f)
    Angles = rng.uniform(0.0, 1.0, (B, T, H, s.a)).astype(f)
    D = rng.standard_normal(H).astype(f) if s.has_d else None
    Qb = (rng.standard_normal((H, N)) * rs).astype(f)
    Kb = (rng.standard_normal((H, N)) * rs).astype(f)
    Z = rng.standard_normal((B, T, H, P)).astype(f) if s.has_z else None
    return dict(Q=Q, K=K, V=V, ADT=ADT, DT=DT, Trap=Trap, Q_bias=Qb, K_bias=Kb, Angles=Angles, D=D, Z=Z)


def mamba3_siso_bytes(s: Mamba3SisoShape) -> int:
    B, T, H, P, N = s.batch, s.seqlen, s.nheads, s.headdim, s.dstate
    return 4 * (2 * B * T * s.hq * N + 2 * B * T * H * P + (B * T * H * P if s.has_z else 0)
                + B * T * H * s.a + 3 * B * H * T + 2 * H * N + (H if s.has_d else 0))


# ---------------------------------------------------------------------------
# Named configurations (the benchmark's and the parity suite's)
# ---------------------------------------------------------------------------

SS_CPU = SelectiveScanShape(batch=1, dim=256, seqlen=512, dstate=16)           # CPU-runnable case
SS_2P8B = SelectiveScanShape(batch=8, dim=5120, seqlen=2048, dstate=16)         # Mamba-2.8B layer shape
GDN2_MAIN = GatedDeltaNet2Shape(batch=4, seqlen=4096, nheads=16, dk=128, dv=128, initial_state=True)
GDN2_LONG = GatedDeltaNet2Shape(batch=1, seqlen=16384, nheads=8, dk=256, dv=256, initial_state=False)
GDN2_WIDEK = GatedDeltaNet2Shape(batch=2, seqlen=2048, nheads=4, dk=320, dv=64, initial_state=True)
GDN2_V65 = GatedDeltaNet2Shape(batch=4, seqlen=4096, nheads=16, dk=128, dv=65, initial_state=True)
# few heads: 32 column-tile workgroups, the sequence-split path
GDN2_FEW = GatedDeltaNet2Shape(batch=1, seqlen=8192, nheads=4, dk=128, dv=128, initial_state=True)
M3_MAIN = Mamba3SisoShape(batch=4, seqlen=4096, nheads=32, headdim=64, dstate=128, angles=64,
                          has_d=True, has_z=False)

NAMED = {
    "selective_scan_b1_d256_l512_n16": SS_CPU,
    "selective_scan_b8_d5120_l2048_n16": SS_2P8B,
    "gated_deltanet2_b4_t4096_h16_k128_v128": GDN2_MAIN,
    "gated_deltanet2_b1_t16384_h8_k256_v256": GDN2_LONG,
    "gated_deltanet2_b2_t2048_h4_k320_v64": GDN2_WIDEK,
    "gated_deltanet2_b4_t4096_h16_k128_v65": GDN2_V65,
    "gated_deltanet2_b1_t8192_h4_k128_v128": GDN2_FEW,
    "mamba3_siso_b4_t4096_h32_p64_n128": M3_MAIN,
}
