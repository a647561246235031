"""Decode step with the reference's ``rnn_step`` contract (torch tensors on a
ROCm device).

``rnn_step_hip(carry, t_inputs, B_bias, C_bias, D)`` mirrors the closure
``rnn_step(carry, t_inputs)`` inside Mamba3SSM.__call_rnn__
(src/base_model/models/mamba3.py:498-562) vmapped over batch: carry =
(theta (B,H,R), ssm (B,H,P,N), k_prev (B,H,N), v_prev (B,H,P)) in float32,
t_inputs = (x_t, z_t, B_t, C_t, adt_t, dt_t, trap_t, angle_t) with trap_t
already through the sigmoid (mamba3.py:489).  The carry is updated in place
(the aliasing XLA gives a scan carry) and returned with y_t (B,H,P).  The mode
knobs read the same environment variables with the same validation as the
reference (mamba3.py:28-45).
"""
from __future__ import annotations

import os
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

_IO = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def recurrent_diagonal_mode() -> str:
    mode = os.environ.get("MAMBA3_RECURRENT_DIAGONAL_MODE", "current")
    if mode not in {"current", "legacy_double"}:
        raise ValueError("MAMBA3_RECURRENT_DIAGONAL_MODE must be current or legacy_double")
    return mode


def recurrent_angle_mode() -> str:
    mode = os.environ.get("MAMBA3_RECURRENT_ANGLE_MODE", "wrapped")
    if mode not in {"wrapped", "legacy_unbounded"}:
        raise ValueError("MAMBA3_RECURRENT_ANGLE_MODE must be wrapped or legacy_unbounded")
    return mode


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def rnn_step_hip(carry: Sequence[torch.Tensor], t_inputs: Sequence[torch.Tensor],
                 B_bias: torch.Tensor, C_bias: torch.Tensor, D: Optional[torch.Tensor],
                 angle_mode: Optional[str] = None, diag_mode: Optional[str] = None,
                 out_dtype: torch.dtype = torch.float32
                 ) -> Tuple[Tuple[torch.Tensor, ...], torch.Tensor]:
    theta, ssm, kprev, vprev = carry
    x, z, Bt, Ct, adt, dt, trap, ang = t_inputs
    angle_mode = angle_mode or recurrent_angle_mode()
    diag_mode = diag_mode or recurrent_diagonal_mode()
    from .ops import mamba3_contraction_precision_mode
    mamba3_contraction_precision_mode()     # the reference's decode reads it too (mamba3.py:545)
    _req(angle_mode in ("wrapped", "legacy_unbounded"), "angle_mode must be wrapped or legacy_unbounded")
    _req(diag_mode in ("current", "legacy_double"), "diag_mode must be current or legacy_double")
    B, H, P, N = ssm.shape
    R = theta.shape[-1]
    for name, t in (("theta", theta), ("ssm", ssm), ("k_prev", kprev), ("v_prev", vprev)):
        _req(t.is_cuda, f"{name} must be a ROCm device tensor; the HIP decode has no CPU path")
        _req(t.dtype == torch.float32 and t.is_contiguous(),
             f"carry {name} must be a contiguous float32 tensor (it is updated in place)")
    _req(tuple(theta.shape) == (B, H, R), f"theta must be {(B, H, R)}, got {tuple(theta.shape)}")
    _req(tuple(kprev.shape) == (B, H, N), f"k_prev must be {(B, H, N)}, got {tuple(kprev.shape)}")
    _req(tuple(vprev.shape) == (B, H, P), f"v_prev must be {(B, H, P)}, got {tuple(vprev.shape)}")
    _req(tuple(x.shape) == (B, H, P), f"x_t must be {(B, H, P)}, got {tuple(x.shape)}")
    if z is not None:
        _req(tuple(z.shape) == (B, H, P), f"z_t must be {(B, H, P)}, got {tuple(z.shape)}")
    _req(tuple(Bt.shape) == (B, H, N) and tuple(Ct.shape) == (B, H, N), "B_t and C_t must be (B, H, N)")
    for name, t in (("adt_t", adt), ("dt_t", dt), ("trap_t", trap)):
        _req(tuple(t.shape) == (B, H), f"{name} must be {(B, H)}, got {tuple(t.shape)}")
    _req(tuple(ang.shape) == (B, H, R), f"angle_t must be {(B, H, R)}, got {tuple(ang.shape)}")
    _req(tuple(B_bias.shape) == (H, N) and tuple(C_bias.shape) == (H, N), "biases must be (H, N)")
    in_dt = x.dtype
    _req(in_dt in _IO and out_dtype in _IO, "x_t and y dtypes must be float32 or bfloat16")
    f32 = lambda t: t.to(torch.float32).contiguous()  # noqa: E731
    cin = lambda t: None if t is None else t.to(in_dt).contiguous()  # noqa: E731
    x, z, Bt, Ct = cin(x), cin(z), cin(Bt), cin(Ct)
    adt, dt, trap, ang, B_bias, C_bias = (f32(t) for t in (adt, dt, trap, ang, B_bias, C_bias))
    Dv = None if D is None else f32(D)
    y = torch.empty((B, H, P), dtype=out_dtype, device=ssm.device)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = _lib.load().m3_decode_step(
        p(theta), p(ssm), p(kprev), p(vprev), p(x), p(z), p(Bt), p(Ct), p(adt), p(dt), p(trap),
        p(ang), p(B_bias), p(C_bias), p(Dv), p(y), B, H, N, P, R, _IO[in_dt], _IO[out_dtype],
        1 if angle_mode == "wrapped" else 0, 1 if diag_mode == "legacy_double" else 0,
        torch.cuda.current_stream(ssm.device).cuda_stream)
    _lib.check(rc, "m3_decode_step")
    return (theta, ssm, kprev, vprev), y
