"""Independent formulations that pin the oracle (test infrastructure only).

None of these reuse ``oracle.mamba3_ref``: rotation is done with complex
numbers, angles and decays are accumulated with plain Python floats, and the
scan is evaluated in its quadratic (attention) form by brute force.  A dropped
term, a wrong sign, a swapped rope pair or a shifted trapezoid weight in the
restatement makes one of them disagree.
"""
from __future__ import annotations

import math

import numpy as np


def _rot(x, theta):
    """Rotate interleaved pairs of x by theta[j] (j < len(theta)) as complex
    multiplication (x0 + i x1) * e^{i theta}; later pairs pass through."""
    x = np.asarray(x, dtype=np.float64)
    out = x.copy()
    for j, th in enumerate(theta):
        zc = complex(x[2 * j], x[2 * j + 1]) * complex(math.cos(th), math.sin(th))
        out[2 * j], out[2 * j + 1] = zc.real, zc.imag
    return out


def _sig(v):
    return 1.0 / (1.0 + math.exp(-v))


def quadratic_form(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z):
    """Brute-force attention form of the Mamba3 SISO scan, float64.

    y_t = silu(z_t) * [ sum_{s<t} (rot(q_t+qb, Th_t) . rot(k_s+kb, Th_s))
                          * e^{A_t - A_s} * scale_s * v_s
                        + (D + gamma_t (q_t+qb).(k_t+kb)) v_t ]
    with Th_t = sum_{i<=t} tanh(angles_i) pi dt_i, A_t = sum_{i<=t} ADT_i,
    gamma_t = dt_t sig(trap_t), scale_s = gamma_s + dt_{s+1}(1 - sig(trap_{s+1}))
    (0 past the end).  Shapes as the oracle entry (unbatched).  O(L^2 H N).
    """
    L, H, N = Q.shape
    P = V.shape[2]
    R = angles.shape[2]
    y = np.zeros((L, H, P))
    for h in range(H):
        th = [0.0] * R
        A = 0.0
        qr, kr, Acum, scale, diag = [], [], [], [], []
        for t in range(L):
            dt = float(DT[h, t])
            for r in range(R):
                th[r] += math.tanh(float(angles[t, h, r])) * math.pi * dt
            A += float(ADT[h, t])
            qb = np.asarray(Q[t, h], np.float64) + np.asarray(Q_bias[h], np.float64)
            kb = np.asarray(K[t, h], np.float64) + np.asarray(K_bias[h], np.float64)
            g = dt * _sig(float(Trap[h, t]))
            sh = 0.0
            if t + 1 < L:
                sh = float(DT[h, t + 1]) * (1.0 - _sig(float(Trap[h, t + 1])))
            qr.append(_rot(qb, th))
            kr.append(_rot(kb, th))
            Acum.append(A)
            scale.append(g + sh)
            diag.append(g * float(np.dot(qb, kb)))
        for t in range(L):
            acc = np.zeros(P)
            for s in range(t):
                w = float(np.dot(qr[t], kr[s])) * math.exp(Acum[t] - Acum[s]) * scale[s]
                acc += w * np.asarray(V[s, h], np.float64)
            d = 0.0 if D is None else float(D[h])
            acc += (d + diag[t]) * np.asarray(V[t, h], np.float64)
            if Z is not None:
                zz = np.asarray(Z[t, h], np.float64)
                acc *= zz / (1.0 + np.exp(-zz))
            y[t, h] = acc
    return y


def seq_inputs_from_scan_args(Q, K, V, ADT, DT, Trap, angles, Z):
    """Map the chunked-scan arguments onto the decode recurrence's per-token
    inputs (the model feeds both from the same _preprocess, mamba3.py:485-489):
    x=V, z=Z, B=K, C=Q, adt=ADT^T, dt=DT^T, trap=sigmoid(Trap)^T, angle=angles."""
    trap = 1.0 / (1.0 + np.exp(-np.asarray(Trap, np.float64)))
    z = np.zeros_like(V) if Z is None else Z
    return (np.asarray(V, np.float64), np.asarray(z, np.float64),
            np.asarray(K, np.float64), np.asarray(Q, np.float64),
            np.asarray(ADT, np.float64).T, np.asarray(DT, np.float64).T, trap.T,
            np.asarray(angles, np.float64))
