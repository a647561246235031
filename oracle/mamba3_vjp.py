"""Gradients of the reference Mamba3 SISO scan (CPU oracle, test-only).

The reference pins its backward kernels against ``jax.grad`` of the XLA scan
``mamba3_ssd_chunked_jax`` (tests/unit/test_mamba3_pallas_ssd.py:108-128, bar
2e-5 relative per gradient at f32).  JAX is not installed here, so this module
restates the same forward in torch, float64 on the CPU, operation for operation
as ``oracle.mamba3_ref.mamba3_ssd_chunked`` (mamba3_jax.py:62-419), and
differentiates it with torch autograd.  The forward restatement is pinned
against the numpy oracle; the gradients are pinned by central finite
differences on small problems and by chunk-size invariance
(``tests/test_oracle_vjp.py``).

Gradient order and shapes follow the reference's custom_vjp
(mamba3_ops.py:821-902): (dQ, dK, dV, dADT, dDT, dTrap, dQ_bias, dK_bias,
dAngles, dD, dZ), each shaped like its input; dD and dZ are None when D and Z
are absent.  With Hqk < H (GQA) the Q and K gradients are summed over the
value heads that share a Q/K head, which autograd does through the head index.
"""
from __future__ import annotations

import math

import numpy as np

NAMES = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")


def _torch():
    import torch
    return torch


def _segsum(x):
    """mamba3_jax.py:62-82: cumsum differences, -inf strictly above the diagonal."""
    torch = _torch()
    T = x.shape[-1]
    cs = torch.cumsum(x, dim=-1)
    out = cs[..., :, None] - cs[..., None, :]
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    return out.masked_fill(~mask, -math.inf)


def _rope(x, cos_a, sin_a):
    """mamba3_jax.py:85-121: rotate interleaved pairs (2j, 2j+1), j < R."""
    torch = _torch()
    d_half = x.shape[-1] // 2
    R = cos_a.shape[-1]
    pairs = x.reshape(*x.shape[:-1], d_half, 2)
    x0, x1 = pairs[..., 0], pairs[..., 1]
    if R < d_half:
        pad = d_half - R
        cos_a = torch.cat([cos_a, torch.ones(*cos_a.shape[:-1], pad, dtype=x.dtype)], dim=-1)
        sin_a = torch.cat([sin_a, torch.zeros(*sin_a.shape[:-1], pad, dtype=x.dtype)], dim=-1)
    out0 = x0 * cos_a - x1 * sin_a
    out1 = x0 * sin_a + x1 * cos_a
    return torch.stack([out0, out1], dim=-1).reshape(x.shape)


def scan(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, chunk_size=64):
    """Differentiable forward, batched torch float64 tensors in the
    ``mamba3_siso_triton`` argument order (mamba3_ops.py:1116-1119):
    Q, K (B, L, Hqk, N); V, Z (B, L, H, P); ADT, DT, Trap (B, H, L); Q_bias,
    K_bias (H, N); Angles (B, L, H, R); D (H,) or None; Z or None.
    Returns y (B, L, H, P).  Same operations as mamba3_jax.py:236-419."""
    torch = _torch()
    Bsz, L, Hqk, N = Q.shape
    H, P = V.shape[2], V.shape[3]
    CS = chunk_size
    idx = torch.arange(H) // (H // Hqk)
    Q, K = Q[:, :, idx], K[:, :, idx]                                   # GQA expansion
    # phase 1 (mamba3_jax.py:124-170, 272-287)
    scaled = torch.tanh(Angles) * math.pi * DT.transpose(1, 2)[..., None]
    cs = torch.cumsum(scaled, dim=1)
    th = cs - 2.0 * math.pi * torch.floor(cs / (2.0 * math.pi))
    cos_a, sin_a = torch.cos(th), torch.sin(th)
    sig = torch.sigmoid(Trap)
    gamma = DT * sig
    shifted = torch.nn.functional.pad((DT * (1.0 - sig))[..., 1:], (0, 1))
    scale = gamma + shifted                                             # (B, H, L)
    Qb = Q + Q_bias
    Kb = K + K_bias
    QK_dot = (Qb * Kb).sum(-1) * gamma.transpose(1, 2)                  # (B, L, H)
    Q_rot = _rope(Qb, cos_a, sin_a)
    K_sc = _rope(Kb, cos_a, sin_a) * scale.transpose(1, 2)[..., None]
    # padding and chunking (mamba3_jax.py:293-324)
    pad = (CS - L % CS) % CS
    padL = lambda x: torch.nn.functional.pad(x, (0, 0) * (x.dim() - 2) + (0, pad))  # noqa: E731
    Qc, Kc, Vc = padL(Q_rot), padL(K_sc), padL(V)
    QKc = torch.nn.functional.pad(QK_dot, (0, 0, 0, pad))
    ADTc = torch.nn.functional.pad(ADT, (0, pad))
    nc = (L + pad) // CS
    Qc = Qc.reshape(Bsz, nc, CS, H, N)
    Kc = Kc.reshape(Bsz, nc, CS, H, N)
    Vc = Vc.reshape(Bsz, nc, CS, H, P)
    QKc = QKc.reshape(Bsz, nc, CS, H)
    ADTc = ADTc.reshape(Bsz, H, nc, CS)
    # phase 3 (mamba3_jax.py:371-393)
    A_cum = torch.cumsum(ADTc, dim=-1)
    Lmat = torch.exp(_segsum(ADTc))
    strict = torch.tril(torch.ones(CS, CS, dtype=torch.bool), diagonal=-1)
    Lmat = torch.where(strict, Lmat, torch.zeros((), dtype=Lmat.dtype))
    S = torch.einsum("bclhn,bcshn->bhcls", Qc, Kc)
    Y_diag = torch.einsum("bhcls,bcshp->bclhp", S * Lmat, Vc)
    # phases 4-6 (mamba3_jax.py:177-233): chunk states, dense cross-chunk pass, output
    decay_states = torch.exp(A_cum[..., -1:] - A_cum)                  # (B, H, nc, CS)
    Vd = Vc * decay_states.permute(0, 2, 3, 1)[..., None]
    states = torch.einsum("bcshp,bcshn->bchpn", Vd, Kc)
    states = torch.cat([torch.zeros_like(states[:, :1]), states], dim=1)
    A_end = torch.nn.functional.pad(A_cum[..., -1], (1, 0))            # (B, H, nc+1)
    decay_chunk = torch.exp(_segsum(A_end))                            # (B, H, nc+1, nc+1)
    new_states = torch.einsum("bhzc,bchpn->bzhpn", decay_chunk, states)
    states_in = new_states[:, :-1]
    Qd = Qc * torch.exp(A_cum).permute(0, 2, 3, 1)[..., None]
    Y_off = torch.einsum("bclhn,bchpn->bclhp", Qd, states_in)
    # phase 7 (mamba3_jax.py:402-419)
    Dv = torch.zeros(H, dtype=V.dtype) if D is None else D
    Y = Y_diag + Y_off + (Dv[:, None] + QKc[..., None]) * Vc
    if Z is not None:
        Zc = padL(Z).reshape(Bsz, nc, CS, H, P)
        Y = Y * (Zc * torch.sigmoid(Zc))
    return Y.reshape(Bsz, nc * CS, H, P)[:, :L]


def vjp(d, cot, chunk_size=64, no_d=False, no_z=False):
    """Gradients of sum(scan(inputs) * cot) w.r.t. every input.

    ``d`` is an inputs dict of numpy arrays as made by ``oracle.inputs.scan_inputs``
    (keys Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z); ``cot`` (B, L, H, P).
    Returns (y, grads) as float64 numpy arrays, grads in NAMES order (None for an
    absent D or Z)."""
    torch = _torch()
    t = {}
    for k in NAMES:
        if (k == "D" and no_d) or (k == "Z" and no_z):
            t[k] = None
            continue
        t[k] = torch.tensor(np.asarray(d[k], dtype=np.float64), requires_grad=True)
    y = scan(*(t[k] for k in NAMES), chunk_size=chunk_size)
    (y * torch.tensor(np.asarray(cot, dtype=np.float64))).sum().backward()
    grads = tuple(None if t[k] is None else t[k].grad.numpy() for k in NAMES)
    return y.detach().numpy(), grads


def cotangent(B, L, H, P, seed):
    """Seeded N(0, 1) output cotangent (the reference draws one per test,
    test_mamba3_pallas_ssd.py:111)."""
    return np.random.default_rng(seed).standard_normal((B, L, H, P)).astype(np.float32)
