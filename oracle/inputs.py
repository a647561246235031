"""Seeded synthetic inputs for the scan and decode configurations (test-only).

Distributions (the benchmark configurations, mapped onto the call signature
``mamba3_siso_triton(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z)``,
src/base_model/models/mamba3_ops.py:1116-1119):
  V = x ~ N(0,1); Z ~ N(0,1); DT = softplus(N(-2, 0.5)) per (b,h,t);
  A_h = -exp(U[ln 1, ln 16]) per head, ADT = A_h * DT;
  Q = C, K = B ~ N(0,1)/sqrt(N); Q_bias, K_bias ~ N(0,1)/sqrt(N) per head;
  D ~ N(0,1) per head; Angles ~ U[-pi, pi]; Trap ~ U(0,1) (pre-sigmoid input).
``numpy.random.default_rng(seed)`` only, so inputs do not depend on any
framework.  bf16 inputs are float32 draws rounded to nearest-even bf16.
"""
from __future__ import annotations

import numpy as np


def softplus(x):
    return np.logaddexp(0.0, x)


def bf16_round(x):
    """Round float32 values to the nearest bf16 (ties to even); returns float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    u = (u + 0x7FFF + lsb) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def bf16_bits(x):
    """uint16 bit patterns of bf16_round(x)."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def scan_inputs(B, L, H, N, P, R, seed, Hqk=None, bf16=False):
    """Batched scan inputs: Q, K (B,L,Hqk,N); V, Z (B,L,H,P); ADT, DT, Trap
    (B,H,L); Angles (B,L,H,R); Q_bias, K_bias (H,N); D (H,).  All float32;
    with ``bf16`` the Q, K, V, Z values are bf16-representable."""
    Hqk = H if Hqk is None else Hqk
    rng = np.random.default_rng(seed)
    f = np.float32
    sN = 1.0 / np.sqrt(N)
    Q = (rng.standard_normal((B, L, Hqk, N), dtype=f) * sN).astype(f)
    K = (rng.standard_normal((B, L, Hqk, N), dtype=f) * sN).astype(f)
    V = rng.standard_normal((B, L, H, P), dtype=f)
    Z = rng.standard_normal((B, L, H, P), dtype=f)
    DT = softplus(rng.normal(-2.0, 0.5, size=(B, H, L))).astype(f)
    A = -np.exp(rng.uniform(np.log(1.0), np.log(16.0), size=(H,))).astype(f)
    ADT = (A[None, :, None] * DT).astype(f)
    Trap = rng.uniform(0.0, 1.0, size=(B, H, L)).astype(f)
    Angles = rng.uniform(-np.pi, np.pi, size=(B, L, H, R)).astype(f)
    Q_bias = (rng.standard_normal((H, N), dtype=f) * sN).astype(f)
    K_bias = (rng.standard_normal((H, N), dtype=f) * sN).astype(f)
    D = rng.standard_normal((H,), dtype=f)
    if bf16:
        Q, K, V, Z = (bf16_round(a) for a in (Q, K, V, Z))
    return dict(Q=Q, K=K, V=V, ADT=ADT, DT=DT, Trap=Trap, Q_bias=Q_bias,
                K_bias=K_bias, Angles=Angles, D=D, Z=Z)


def decode_inputs(B, H, N, P, R, steps, seed, bf16=True):
    """Decode carry and per-step inputs (config 4 distributions).

    carry: theta (B,H,R) ~ U[0,2pi); h (B,H,P,N) ~ N(0, 0.1); k_prev (B,H,N)
    ~ N(0,1)/sqrt(N); v_prev (B,H,P) ~ N(0,1).  Per step (leading ``steps``
    axis): x, z (B,H,P) ~ N(0,1); Bt, Ct (B,H,N) ~ N(0,1)/sqrt(N); dt =
    softplus(N(-2,0.5)); adt = A_h dt with A_h = -exp(U[0, ln 16]); trap =
    sigmoid(U(0,1)) (post-sigmoid, as rnn_step takes it); angle ~ U[-pi,pi].
    Biases B_bias, C_bias (H,N) ~ N(0,1)/sqrt(N); D (H,) ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    f = np.float32
    sN = 1.0 / np.sqrt(N)
    theta = rng.uniform(0.0, 2 * np.pi, size=(B, H, R)).astype(f)
    h = (rng.standard_normal((B, H, P, N), dtype=f) * 0.1).astype(f)
    k_prev = (rng.standard_normal((B, H, N), dtype=f) * sN).astype(f)
    v_prev = rng.standard_normal((B, H, P), dtype=f)
    x = rng.standard_normal((steps, B, H, P), dtype=f)
    z = rng.standard_normal((steps, B, H, P), dtype=f)
    Bt = (rng.standard_normal((steps, B, H, N), dtype=f) * sN).astype(f)
    Ct = (rng.standard_normal((steps, B, H, N), dtype=f) * sN).astype(f)
    dt = softplus(rng.normal(-2.0, 0.5, size=(steps, B, H))).astype(f)
    A = -np.exp(rng.uniform(0.0, np.log(16.0), size=(H,))).astype(f)
    adt = (A[None, None, :] * dt).astype(f)
    trap = (1.0 / (1.0 + np.exp(-rng.uniform(0.0, 1.0, size=(steps, B, H))))).astype(f)
    ang = rng.uniform(-np.pi, np.pi, size=(steps, B, H, R)).astype(f)
    B_bias = (rng.standard_normal((H, N), dtype=f) * sN).astype(f)
    C_bias = (rng.standard_normal((H, N), dtype=f) * sN).astype(f)
    D = rng.standard_normal((H,), dtype=f)
    if bf16:
        x, z, Bt, Ct = (bf16_round(a) for a in (x, z, Bt, Ct))
    return dict(theta=theta, h=h, k_prev=k_prev, v_prev=v_prev, x=x, z=z, Bt=Bt,
                Ct=Ct, adt=adt, dt=dt, trap=trap, ang=ang, B_bias=B_bias,
                C_bias=C_bias, D=D)
