"""Numpy restatement of the Mamba3 mixer layer (CPU oracle, test-only).

Mamba3SSM.__call__ of src/base_model/models/mamba3.py with the fused path's
shared B/C (shared_bc=True, :356): in_proj, the split of :212-219, BCNorm
(flax RMSNorm, eps 1e-6, statistics in float32 or wider) of :240-242, the decay
of :251-254, the scan (oracle.mamba3_ref, with Q = C and K = B shared over heads
and the angle rates repeated), and _post_norm_and_project of :281-331 (one
device).  With ``bf16=True`` the values are rounded to bf16 where the reference's
bf16 layer holds them in bf16: the projection output, the normalised B and C
(the kernels' operands), the scan output, y * rsqrt in y's dtype, the product
with the norm scale before out_proj, and the out_proj result.  Pinned by
tests/test_oracle_layer.py.
"""
from __future__ import annotations

import math

import numpy as np

from . import inputs as I
from . import mamba3_ref as M

EPS = 1e-6


def softplus(x):
    """jax.nn.softplus = logaddexp(x, 0)."""
    return np.logaddexp(x, 0.0)


def rmsnorm(x, scale, eps=EPS):
    """flax nn.RMSNorm over the last axis: x * rsqrt(mean(x^2) + eps) * scale."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * scale


def dims(d_model, d_state=128, expand=2, headdim=64, rope_fraction=0.5):
    """Head count, head dim, rope pairs and in_proj width as Mamba3SSM.setup
    computes them (mamba3.py:112-142)."""
    d_inner_target = expand * d_model
    hd = min(headdim, d_inner_target)
    nh = max(1, d_inner_target // hd)
    split = int(d_state * rope_fraction)
    split -= split % 2
    R = split // 2
    d_in_proj = 2 * nh * hd + 2 * d_state + 3 * nh + R
    return nh, hd, R, d_in_proj


def init_params(d_model, seed, d_state=128, expand=2, headdim=64, rope_fraction=0.5,
                dt_min=0.001, dt_max=0.1, perturb=True):
    """Random parameters with the reference's initialisers (mamba3.py:145-183):
    Dense kernels N(0, 1/fan_in), dt_bias the inverse softplus of log-uniform
    dt in [dt_min, dt_max], biases/D/norm scales ones.  ``perturb`` moves the
    ones by N(0, 0.1) so that every parameter is exercised by the parity tests."""
    rng = np.random.default_rng(seed)
    nh, hd, R, dproj = dims(d_model, d_state, expand, headdim, rope_fraction)
    di = nh * hd
    f = np.float32
    u = rng.uniform(size=nh)
    dt = np.exp(u * (math.log(dt_max) - math.log(dt_min)) + math.log(dt_min))
    dt = np.maximum(dt, 1e-4)
    p = dict(
        in_proj=(rng.standard_normal((d_model, dproj)) / math.sqrt(d_model)).astype(f),
        dt_bias=(dt + np.log(-np.expm1(-dt))).astype(f),
        B_bias=np.ones((nh, d_state), f), C_bias=np.ones((nh, d_state), f),
        B_norm=np.ones(d_state, f), C_norm=np.ones(d_state, f), D=np.ones(nh, f),
        out_norm=np.ones(di, f),
        out_proj=(rng.standard_normal((di, d_model)) / math.sqrt(di)).astype(f),
    )
    if perturb:
        for k in ("B_bias", "C_bias", "B_norm", "C_norm", "D", "out_norm"):
            p[k] = (p[k] + 0.1 * rng.standard_normal(p[k].shape)).astype(f)
    return p


def split_proj(proj, di, N, nh):
    """The in_proj output split [z, x, B, C, dd_dt, dd_A, trap, angles] along the last
    axis, widths [di, di, N, N, nh, nh, nh, R] (mamba3.py:212-219)."""
    cut = np.cumsum([di, di, N, N, nh, nh, nh])
    return np.split(proj, cut, axis=-1)


def decay(dd_dt, dd_A, dt_bias, A_floor):
    """(A, DT): A = clip(-softplus(dd_A), max=-A_floor), DT = softplus(dd_dt + dt_bias)
    (mamba3.py:251-254)."""
    A = np.minimum(-softplus(dd_A), -A_floor)
    DT = softplus(dd_dt + dt_bias)
    return A, DT


def layer_forward(p, x, d_state=128, headdim=64, rope_fraction=0.5, A_floor=1e-4, chunk_size=64,
                  bf16=False):
    """Mamba3SSM.__call__ on x (B, L, d_model) -> (B, L, d_model), float64 math."""
    rnd = I.bf16_round if bf16 else (lambda a: a)
    r = lambda a: np.asarray(rnd(np.asarray(a, np.float32)), np.float64) if bf16 else np.asarray(a, np.float64)  # noqa: E731
    B, L, d_model = x.shape
    N = d_state
    nh, hd, R, dproj = dims(d_model, d_state, 2, headdim, rope_fraction)
    di = nh * hd
    xin = r(x)
    proj = r(xin @ r(p["in_proj"]))                                     # in_proj (mamba3.py:210)
    z, xv, Bm, Cm, dd_dt, dd_A, trap, ang = split_proj(proj, di, N, nh)  # :212-219
    Bn = r(rmsnorm(Bm, p["B_norm"]))                                    # BCNorm, :240-242
    Cn = r(rmsnorm(Cm, p["C_norm"]))
    A, DT = decay(dd_dt, dd_A, p["dt_bias"], A_floor)                   # :251-254
    ADT = A * DT
    ang_rep = np.repeat(ang[:, :, None, :], nh, axis=2)                 # (B, L, nh, R)
    y = M.mamba3_ssd_chunked_batched(
        Cn[:, :, None, :], Bn[:, :, None, :], xv.reshape(B, L, nh, hd),
        np.transpose(ADT, (0, 2, 1)), np.transpose(DT, (0, 2, 1)), np.transpose(trap, (0, 2, 1)),
        ang_rep, p["C_bias"], p["B_bias"], p["D"], z.reshape(B, L, nh, hd), chunk_size=chunk_size)
    y = r(y.reshape(B, L, di))
    rms_inv = 1.0 / np.sqrt(np.mean(y * y, axis=-1, keepdims=True) + EPS)   # :293-303
    yn = r(y * r(rms_inv))
    yn = r(yn * p["out_norm"])
    return r(yn @ r(p["out_proj"]))                                     # :314-325
