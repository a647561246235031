"""Numpy restatement of the reference Mamba3 SISO scan (CPU oracle, test-only).

Follows the reference operation for operation; every function cites the
reference lines it restates (paths relative to the sigma-0 repository root).
The arithmetic type is a parameter: float64 (default) is the exact-math
yardstick the GPU kernels are compared against; float32 reproduces the
reference's own arithmetic class (XLA, ``precision=HIGHEST``) and is what the
CPU baseline times.

Parity of this module is pinned by ``oracle.pins`` (brute-force quadratic
form, token-by-token recurrence) and by the invariants exercised in
``tests/test_oracle.py``.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "segsum", "apply_rope", "angle_dt_cumsum", "trapezoid_gamma_scale",
    "preprocess_and_chunk", "phases_4_5_6", "mamba3_ssd_chunked",
    "mamba3_ssd_chunked_batched", "rnn_step", "rnn_scan",
]


def _c(x, dt):
    return np.asarray(x, dtype=dt)


def segsum(x):
    """Pairwise cumsum differences, -inf strictly above the diagonal.

    Restates mamba3_jax.py:62-82: cumsum along the last axis, then
    ``cs[..., :, None] - cs[..., None, :]`` masked with ``tril``.
    """
    T = x.shape[-1]
    cs = np.cumsum(x, axis=-1)
    out = cs[..., :, None] - cs[..., None, :]
    mask = np.tril(np.ones((T, T), dtype=bool))
    return np.where(mask, out, -np.inf).astype(x.dtype)


def apply_rope(x, cos_angles, sin_angles):
    """Rotate interleaved pairs (2j, 2j+1) for j < R; the rest passes through.

    Restates mamba3_jax.py:85-121 (cos padded with 1, sin with 0 when
    R < d/2).
    """
    d = x.shape[-1]
    d_half = d // 2
    pairs = x.reshape(*x.shape[:-1], d_half, 2)
    x0, x1 = pairs[..., 0], pairs[..., 1]
    d_rope = cos_angles.shape[-1]
    if d_rope < d_half:
        pad = [(0, 0)] * (cos_angles.ndim - 1) + [(0, d_half - d_rope)]
        cos_angles = np.pad(cos_angles, pad, constant_values=1.0)
        sin_angles = np.pad(sin_angles, pad, constant_values=0.0)
    out0 = x0 * cos_angles - x1 * sin_angles
    out1 = x0 * sin_angles + x1 * cos_angles
    return np.stack([out0, out1], axis=-1).reshape(x.shape)


def angle_dt_cumsum(angles, dt):
    """Theta[l,h,r] = (sum_{i<=l} tanh(angles[i,h,r]) * pi * dt[h,i]) mod 2pi.

    Restates mamba3_jax.py:124-144: one global cumsum over L, then a single
    range reduction ``c - 2pi*floor(c/2pi)``.
    angles: (L, H, R); dt: (H, L) -> (L, H, R).
    """
    f = angles.dtype.type
    PI = f(np.pi)
    TWO_PI = f(2.0) * PI
    scaled = np.tanh(angles) * PI * dt.T[..., None]
    cs = np.cumsum(scaled, axis=0)
    return cs - TWO_PI * np.floor(cs / TWO_PI)


def trapezoid_gamma_scale(DT, Trap):
    """gamma = dt*sigmoid(trap); scale = gamma + shift_left(dt*(1-sigmoid(trap))).

    Restates mamba3_jax.py:147-170 (the shifted term is 0 at t = L-1).
    DT, Trap: (H, L) -> gamma, scale: (H, L).
    """
    one = DT.dtype.type(1.0)
    sig = one / (one + np.exp(-Trap))
    gamma = DT * sig
    dt_sh = np.pad(DT[:, 1:], ((0, 0), (0, 1)))
    sig_sh = np.pad(sig[:, 1:], ((0, 0), (0, 1)))
    shifted = dt_sh * (one - sig_sh)
    return gamma, gamma + shifted


def preprocess_and_chunk(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, Z,
                         chunk_size=64):
    """Phases 1-2: rope angles, trapezoid weights, biases, QK-dot skip,
    rotation, key scaling, padding to a chunk multiple and reshape.

    Restates mamba3_jax.py:236-324 in the same order: bias before the QK dot
    and before rotation (:272-284), K scaled after rotation (:287), L padded
    with zeros (:293-313).
    """
    L, H, N = Q.shape
    P = V.shape[2]
    CS = chunk_size
    th = angle_dt_cumsum(angles, DT)
    cos_a, sin_a = np.cos(th), np.sin(th)
    gamma, scale = trapezoid_gamma_scale(DT, Trap)
    Qb = Q + Q_bias[None, :, :]
    Kb = K + K_bias[None, :, :]
    QK_dot = np.sum(Qb * Kb, axis=-1) * gamma.T              # (L, H)
    Q_rot = apply_rope(Qb, cos_a, sin_a)
    K_rot = apply_rope(Kb, cos_a, sin_a)
    K_scaled = K_rot * scale.T[..., None]

    pad = (CS - L % CS) % CS

    def padL(x):
        if pad == 0:
            return x
        return np.pad(x, [(0, pad)] + [(0, 0)] * (x.ndim - 1))

    Q_rot, K_scaled, Vp, Zp, QKp = (padL(a) for a in (Q_rot, K_scaled, V, Z, QK_dot))
    ADTp = np.pad(ADT, ((0, 0), (0, pad))) if pad else ADT
    Lp = L + pad
    nc = Lp // CS
    return (Q_rot.reshape(nc, CS, H, N), K_scaled.reshape(nc, CS, H, N),
            Vp.reshape(nc, CS, H, P), Zp.reshape(nc, CS, H, P),
            QKp.reshape(nc, CS, H), ADTp.reshape(H, nc, CS), L, Lp)


def phases_4_5_6(Q_c, K_c, V_c, ADT_c, A_cumsum):
    """Per-chunk states, dense cross-chunk pass, state -> output.

    Restates mamba3_jax.py:177-233: phase 4 'cshp,hcs,cshn->chpn' with
    exp(A_end - A_cum); phase 5 the dense segsum over nc+1 chunk states with
    a zero initial state; phase 6 'clhn,chpn,hcl->clhp' with exp(A_cum).
    """
    nc, CS, H, N = Q_c.shape
    P = V_c.shape[-1]
    decay_states = np.exp(A_cumsum[:, :, -1:] - A_cumsum)           # (H, nc, CS)
    Vd = V_c * np.transpose(decay_states, (1, 2, 0))[..., None]      # (nc, CS, H, P)
    states = np.einsum("cshp,cshn->chpn", Vd, K_c, optimize=True)   # (nc, H, P, N)
    init = np.zeros((1, H, P, N), dtype=V_c.dtype)
    states = np.concatenate([init, states], axis=0)                 # (nc+1, H, P, N)
    A_end = np.pad(A_cumsum[:, :, -1], ((0, 0), (1, 0)))            # (H, nc+1)
    decay_chunk = np.exp(segsum(A_end))                             # (H, nc+1, nc+1)
    new_states = np.einsum("hzc,chpn->zhpn", decay_chunk, states, optimize=True)
    states_in = new_states[:-1]                                     # entering each chunk
    Qd = Q_c * np.transpose(np.exp(A_cumsum), (1, 2, 0))[..., None]
    return np.einsum("clhn,chpn->clhp", Qd, states_in, optimize=True)


def mamba3_ssd_chunked(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z,
                       chunk_size=64, dtype=np.float64):
    """Oracle entry: the reference's ``mamba3_ssd_chunked_jax`` (unbatched).

    Restates mamba3_jax.py:327-419 (argument order of :327-331).  Shapes:
    Q, K (L, H, N); V, Z (L, H, P); ADT, DT, Trap (H, L); angles (L, H, R);
    Q_bias, K_bias (H, N); D (H,).  ``D=None`` and ``Z=None`` mean no
    feedthrough and no gate (the Triton bridge's optional forms,
    mamba3_ops.py:200-210).  Returns y (L, H, P) in ``dtype``.
    """
    H = Q.shape[1]
    P = V.shape[2]
    args = [_c(a, dtype) for a in (Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias)]
    Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias = args
    Dv = np.zeros((H,), dtype) if D is None else _c(D, dtype)
    has_z = Z is not None
    Zv = np.zeros(V.shape, dtype) if not has_z else _c(Z, dtype)
    Q_c, K_c, V_c, Z_c, QK_c, ADT_c, L, Lp = preprocess_and_chunk(
        Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, Zv, chunk_size)
    CS = chunk_size
    # phase 3 (mamba3_jax.py:371-393): strictly lower-triangular decayed QK^T V
    A_cum = np.cumsum(ADT_c, axis=-1)                                # (H, nc, CS)
    Lmat = np.exp(segsum(ADT_c))                                     # (H, nc, CS, CS)
    strict = np.tril(np.ones((CS, CS), dtype=bool), k=-1)
    Lmat = np.where(strict[None, None], Lmat, 0.0).astype(dtype)
    S = np.einsum("clhn,cshn->hcls", Q_c, K_c, optimize=True)
    Y_diag = np.einsum("hcls,cshp->clhp", S * Lmat, V_c, optimize=True)
    Y_off = phases_4_5_6(Q_c, K_c, V_c, ADT_c, A_cum)
    # phase 7 (mamba3_jax.py:402-419)
    Y = Y_diag + Y_off
    Y = Y + (Dv[None, None, :, None] + QK_c[..., None]) * V_c
    if has_z:
        one = np.dtype(dtype).type(1.0)
        Y = Y * (Z_c / (one + np.exp(-Z_c)))
    return Y.reshape(Lp, H, P)[:L]


def mamba3_ssd_chunked_batched(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias,
                               D, Z, chunk_size=64, dtype=np.float64, heads=None):
    """Batched form (leading B on every per-sequence input), the way the model
    vmaps the scan (lob_seq_model.py:736-766).  Q, K may carry Hqk < H heads
    (GQA, head h reads qk head h // (H/Hqk), siso_fwd.py:161); they are
    expanded here.  ``heads`` optionally restricts the computation to a subset
    of value heads (the scan is independent per (batch, head))."""
    Bsz, L, Hqk, N = Q.shape
    H = V.shape[2]
    if heads is None:
        heads = np.arange(H)
    heads = np.asarray(heads)
    rep = H // Hqk
    qk_idx = heads // rep
    out = []
    for b in range(Bsz):
        out.append(mamba3_ssd_chunked(
            Q[b][:, qk_idx], K[b][:, qk_idx], V[b][:, heads], ADT[b][heads], DT[b][heads],
            Trap[b][heads], angles[b][:, heads], Q_bias[heads], K_bias[heads],
            None if D is None else D[heads], None if Z is None else Z[b][:, heads],
            chunk_size=chunk_size, dtype=dtype))
    return np.stack(out, axis=0)


def rnn_step(carry, t_inputs, B_bias, C_bias, D, angle_mode="wrapped",
             diag_mode="current", dtype=np.float64):
    """One decode step of the Mamba3 recurrence.

    Restates ``rnn_step`` in mamba3.py:498-562 (modes of :28-45):
      theta += tanh(angle_t)*pi*dt (wrapped mod 2pi unless legacy_unbounded)
      B_rot, C_rot = rope(B_t + B_bias), rope(C_t + C_bias)
      h = e^{adt} h + (1-trap) dt e^{adt} (v_prev (x) k_prev) + trap dt (x_t (x) B_rot)
      y = C_rot . h + D x_t  (+ qk*gamma*x_t under legacy_double);  y *= silu(z_t)
    carry = (theta (..,H,R), h (..,H,P,N), k_prev (..,H,N), v_prev (..,H,P));
    t_inputs = (x_t, z_t, B_t, C_t, adt_t, dt_t, trap_t, angle_t) with trap_t
    already passed through the sigmoid (mamba3.py:489).  Leading batch dims
    are allowed.  Returns (new_carry, y_t).
    """
    f = np.dtype(dtype).type
    ang_s, h, k_prev, v_prev = (_c(a, dtype) for a in carry)
    x_t, z_t, B_t, C_t, adt_t, dt_t, trap_t, angle_t = (_c(a, dtype) for a in t_inputs)
    PI = f(np.pi)
    TWO_PI = f(2.0) * PI
    ang_s = ang_s + np.tanh(angle_t) * PI * dt_t[..., None]
    if angle_mode == "wrapped":
        ang_s = ang_s - TWO_PI * np.floor(ang_s / TWO_PI)
    elif angle_mode != "legacy_unbounded":
        raise ValueError("angle_mode must be wrapped or legacy_unbounded")
    cos_a, sin_a = np.cos(ang_s), np.sin(ang_s)
    B_rot = apply_rope(B_t + _c(B_bias, dtype), cos_a, sin_a)
    C_rot = apply_rope(C_t + _c(C_bias, dtype), cos_a, sin_a)
    decay = np.exp(adt_t)[..., None, None]
    tr = trap_t[..., None, None]
    dte = dt_t[..., None, None]
    h = decay * h
    h = h + (f(1.0) - tr) * dte * decay * (v_prev[..., :, None] * k_prev[..., None, :])
    h = h + tr * dte * (x_t[..., :, None] * B_rot[..., None, :])
    y = np.einsum("...hn,...hpn->...hp", C_rot, h)
    y = y + _c(D, dtype)[..., :, None] * x_t
    if diag_mode == "legacy_double":
        gamma = dt_t * trap_t
        qk = np.sum(C_rot * B_rot, axis=-1)
        y = y + (qk * gamma)[..., None] * x_t
    elif diag_mode != "current":
        raise ValueError("diag_mode must be current or legacy_double")
    y = y * (z_t / (f(1.0) + np.exp(-z_t)))
    return (ang_s, h, B_rot, x_t), y


def rnn_scan(carry, seq_inputs, B_bias, C_bias, D, dtype=np.float64, **modes):
    """``jax.lax.scan(rnn_step)`` over the token axis (mamba3.py:564-568).

    seq_inputs hold a leading L axis: x, z (L, .., H, P); B, C (L, .., H, N);
    adt, dt, trap (L, .., H) with trap post-sigmoid; angle (L, .., H, R).
    Returns (final_carry, y (L, .., H, P)).
    """
    L = seq_inputs[0].shape[0]
    ys = []
    for t in range(L):
        carry, y = rnn_step(carry, tuple(a[t] for a in seq_inputs), B_bias, C_bias, D,
                            dtype=dtype, **modes)
        ys.append(y)
    return carry, np.stack(ys, axis=0)
