"""Prefill entry points with the reference's call signatures (torch tensors on a
ROCm device; torch provides device memory and the stream only).

``mamba3_siso_hip`` keeps the argument order and meaning of the reference's
``mamba3_siso_triton(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z,
chunk_size)`` (src/base_model/models/mamba3_ops.py:1116-1127): unbatched
arrays as ``nn.vmap`` hands them over, or the batched layout of its vmap rule
(:1121-1127, :1052-1110).  ``mamba3_ssd_chunked_hip`` keeps the oracle's
order (src/base_model/models/mamba3_jax.py:327-331).  Shape contracts raise
ValueError with the reference's assert messages
(src/base_model/kernels/mamba3_triton/siso_fwd.py:466-482); the result is
returned in ``V.dtype`` (mamba3_ops.py:273).
"""
from __future__ import annotations

import os
from typing import Optional, Tuple

import torch

from . import _lib

_IO = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def mamba3_contraction_precision_mode() -> str:
    """The reference's contraction-precision contract
    (src/base_model/models/mamba3_jax.py:44-52): MAMBA3_CONTRACTION_PRECISION is
    "highest" (the default; an empty value means the default) or "default", anything
    else raises ValueError with the reference's message.  Read on every call, as there.

    "highest" asks for exact float32 contractions, which is what every kernel here
    computes with float32 I/O (float32 MFMA operands, or float32 arithmetic in the
    token-recurrent kernel, with float32 accumulation).
    "default" lets the reference's XLA path use TF32 on its GPUs; gfx950 has no
    TF32-class matrix instruction and bf16 operands would be coarser than TF32, so it
    runs the same exact float32 contractions, which satisfy a mode that permits less.
    With bf16 I/O the operands are bf16 under either mode, with float32 accumulation
    (the reference's Triton kernel dots in the input dtype, siso_fwd.py:333-345).
    """
    mode = os.environ.get("MAMBA3_CONTRACTION_PRECISION") or "highest"
    if mode not in {"highest", "default"}:
        raise ValueError("MAMBA3_CONTRACTION_PRECISION must be highest or default")
    return mode


_DTYPE_NAMES = {"float32": torch.float32, "bfloat16": torch.bfloat16}


def pallas_compute_dtype(default: torch.dtype = torch.float32) -> torch.dtype:
    """The fused path's operand-dtype knob (src/base_model/models/mamba3_pallas.py:
    112-122): MAMBA3_PALLAS_DTYPE ("float32" or "bfloat16") overrides; unset or
    empty, the layer's compute dtype ``default`` decides; anything else raises
    ValueError with the reference's message.  Read on every call, as there.  The
    kernels here take their MFMA operands in the I/O dtype, so the shared-B/C entry
    points cast Q, K, V and Z to this dtype (float32 accumulation either way) and
    return the output in V's dtype."""
    name = os.environ.get("MAMBA3_PALLAS_DTYPE") or {v: k for k, v in _DTYPE_NAMES.items()}.get(default, "")
    if name not in _DTYPE_NAMES:
        raise ValueError("MAMBA3_PALLAS_DTYPE must be float32 or bfloat16")
    return _DTYPE_NAMES[name]


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a ROCm device tensor (got device {t.device}); "
                         "the Mamba3 HIP operator has no CPU path")


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float32).contiguous()


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _prep(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z):
    """Validate and normalise to the batched contiguous layout of the C ABI."""
    mamba3_contraction_precision_mode()
    unbatched = V.dim() == 3
    if unbatched:
        Q, K, V = Q[None], K[None], V[None]
        ADT, DT, Trap = ADT[None], DT[None], Trap[None]
        Angles = Angles[None]
        if Z is not None and Z.dim() == 3:
            Z = Z[None]
    _req(V.dim() == 4, f"V must be (L, H, P) or (B, L, H, P), got {tuple(V.shape)}")
    B, L, HQ, N = Q.shape
    _, _, H, P = V.shape
    for name, t in (("Q", Q), ("K", K), ("V", V)):
        _dev(t, name)
    _req(L > 0 or B == 0, "Sequence length must be greater than 0")
    _req(tuple(Q.shape) == tuple(K.shape), f"Q and K shape mismatch: {tuple(Q.shape)} vs {tuple(K.shape)}")
    _req(H % HQ == 0, f"nheads ({H}) must be divisible by nheads_qk ({HQ})")
    _req(tuple(V.shape[:2]) == (B, L), f"V shape {tuple(V.shape)} does not match Q {tuple(Q.shape)}")
    _req(tuple(ADT.shape) == (B, H, L), f"ADT must be {(B, H, L)}, got {tuple(ADT.shape)}")
    _req(tuple(DT.shape) == (B, H, L), f"DT must be {(B, H, L)}, got {tuple(DT.shape)}")
    _req(tuple(Trap.shape) == (B, H, L), f"Trap must be {(B, H, L)}, got {tuple(Trap.shape)}")
    _req(tuple(Q_bias.shape) == (H, N), f"Q_bias must be {(H, N)}, got {tuple(Q_bias.shape)}")
    _req(tuple(K_bias.shape) == (H, N), f"K_bias must be {(H, N)}, got {tuple(K_bias.shape)}")
    _req(Angles.dim() == 4 and tuple(Angles.shape[:3]) == (B, L, H),
         f"Angles must be {(B, L, H, '<R>')}, got {tuple(Angles.shape)}")
    R = Angles.shape[-1]
    _req(R <= N // 2, f"headdim_angles ({R}) must be <= headdim_qk // 2 ({N // 2})")
    if D is not None:
        _req(tuple(D.shape) == (H,), f"D must be {(H,)}, got {tuple(D.shape)}")
    if Z is not None:
        _req(tuple(Z.shape) == (B, L, H, P), f"Z must be {(B, L, H, P)}, got {tuple(Z.shape)}")
    dt = V.dtype
    _req(dt in _IO, f"V dtype must be float32 or bfloat16, got {dt}")
    Q, K, V = (t.to(dt).contiguous() for t in (Q, K, V))
    Z = None if Z is None else Z.to(dt).contiguous()
    prepared = dict(
        Q=Q, K=K, V=V, ADT=_f32(ADT), DT=_f32(DT), Trap=_f32(Trap), Q_bias=_f32(Q_bias),
        K_bias=_f32(K_bias), Angles=_f32(Angles), D=None if D is None else _f32(D), Z=Z)
    return prepared, (B, L, H, HQ, N, P, R), unbatched


def _launch(p, dims, chunk_size, out, init=None, fin=None, seq_split=True):
    B, L, H, HQ, N, P, R = dims
    lib = _lib.load()
    io = _IO[p["V"].dtype]
    common = (_ptr(p["Q"]), _ptr(p["K"]), _ptr(p["V"]), _ptr(p["ADT"]), _ptr(p["DT"]),
              _ptr(p["Trap"]), _ptr(p["Q_bias"]), _ptr(p["K_bias"]), _ptr(p["Angles"]),
              _ptr(p["D"]), _ptr(p["Z"]), _ptr(out))
    tail = (B, L, H, HQ, N, P, R, int(chunk_size), io)
    ip = tuple(_ptr(t) for t in init) if init is not None else (None,) * 4
    fp = tuple(_ptr(t) for t in fin) if fin is not None else (None,) * 4
    ws_bytes = lib.m3_chunk_scan_ws_bytes(B, L, H, N, P, R, int(chunk_size), io) if seq_split else 0
    if ws_bytes:
        # few (batch, head) pairs: the sequence is split across compute units; the
        # workspace lives for this call only (torch's caching allocator, same stream)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=p["V"].device)
        rc = lib.m3_chunk_scan_fwd_ws(*common, *ip, *fp, *tail, ws.data_ptr(), ws_bytes, _stream(p["V"]))
    elif init is None and fin is None:
        rc = lib.m3_chunk_scan_fwd(*common, *tail, _stream(p["V"]))
    else:
        rc = lib.m3_chunk_scan_fwd_carry(*common, *ip, *fp, *tail, _stream(p["V"]))
    _lib.check(rc, "m3_chunk_scan_fwd")


def mamba3_siso_hip(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D=None, Z=None,
                    chunk_size: int = 64, seq_split: bool = True) -> torch.Tensor:
    """Mamba3 SISO chunked scan forward on gfx950.

    Same arguments as the reference's mamba3_siso_triton (mamba3_ops.py:1116):
    Q, K (L, Hqk, N); V, Z (L, H, P); ADT, DT, Trap (H, L) with Trap the
    pre-sigmoid logits; Q_bias, K_bias (H, N); Angles (L, H, R) raw rates;
    D (H,) or None; Z or None; or all of them with a leading batch dim.
    Returns Out with V's shape and dtype.  ``seq_split`` lets a launch with few
    (batch, head) pairs split each sequence across compute units (same result up
    to rounding); False forces one pass.
    """
    args = (Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z)
    if torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in args):
        return _Mamba3Siso.apply(int(chunk_size), bool(seq_split), *args)
    return _forward(args, chunk_size, seq_split)


def _forward(args, chunk_size, seq_split):
    p, dims, unbatched = _prep(*args)
    out = torch.empty_like(p["V"])
    if out.numel():
        _launch(p, dims, chunk_size, out, seq_split=seq_split)
    return out[0] if unbatched else out


def _forward_train(args, chunk_size, seq_split):
    """The forward plus the residuals its backward reads (the chunk states and their
    rope angles), as the reference's mamba3_siso_fwd returns them
    (mamba3_ops.py:788-818).  Returns (out, saved); saved is None where the library
    has no saved-state path for the shape (the backward then recomputes)."""
    p, (B, L, H, HQ, N, P, R), unbatched = _prep(*args)
    out = torch.empty_like(p["V"])
    if not out.numel():
        return (out[0] if unbatched else out), None
    lib = _lib.load()
    io = _IO[p["V"].dtype]
    kbwd = 64 if io == _lib.DTYPE_BF16 else 32
    nbytes = lib.m3_chunk_scan_saved_bytes(B, L, H, N, P, R, io)
    if nbytes == 0 or int(chunk_size) % kbwd != 0 or \
            lib.m3_chunk_scan_impl(io, N, P, R, int(chunk_size)) != _lib.IMPL_CHUNKED_MFMA:
        _launch(p, (B, L, H, HQ, N, P, R), chunk_size, out, seq_split=seq_split)
        return (out[0] if unbatched else out), None
    saved = torch.empty(nbytes, dtype=torch.uint8, device=p["V"].device)
    ws_bytes = lib.m3_chunk_scan_ws_bytes(B, L, H, N, P, R, int(chunk_size), io) if seq_split else 0
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=p["V"].device)
    rc = lib.m3_chunk_scan_fwd_train(
        _ptr(p["Q"]), _ptr(p["K"]), _ptr(p["V"]), _ptr(p["ADT"]), _ptr(p["DT"]), _ptr(p["Trap"]),
        _ptr(p["Q_bias"]), _ptr(p["K_bias"]), _ptr(p["Angles"]), _ptr(p["D"]), _ptr(p["Z"]), _ptr(out),
        B, L, H, HQ, N, P, R, int(chunk_size), io, saved.data_ptr(), nbytes,
        ws.data_ptr() if ws_bytes else None, ws_bytes, _stream(p["V"]))
    _lib.check(rc, "m3_chunk_scan_fwd_train")
    return (out[0] if unbatched else out), saved


def mamba3_siso_hip_bwd(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z, dOut,
                        chunk_size: int = 64, saved: Optional[torch.Tensor] = None):
    """Gradients of mamba3_siso_hip's output against every input, given dOut (the
    output cotangent, V's shape).  The reference's backward (mamba3_siso_bwd,
    mamba3_ops.py:821-902) returns the same tuple:
    (dQ, dK, dV, dADT, dDT, dTrap, dQ_bias, dK_bias, dAngles, dD, dZ), each in its
    input's shape; dD and dZ are None when D and Z are.  ``saved``: the residuals of
    the training forward on the same inputs (mamba3_siso_hip_fwd_train); without
    them the chunk states are recomputed from the inputs."""
    p, (B, L, H, HQ, N, P, R), unbatched = _prep(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z)
    io = _IO[p["V"].dtype]
    dO = (dOut[None] if unbatched else dOut).to(p["V"].dtype).contiguous()
    _req(tuple(dO.shape) == (B, L, H, P), f"dOut must be {(B, L, H, P)}, got {tuple(dOut.shape)}")
    dev, dt = p["V"].device, p["V"].dtype
    f32 = dict(device=dev, dtype=torch.float32)
    g = dict(Q=torch.empty_like(p["Q"]), K=torch.empty_like(p["K"]), V=torch.empty_like(p["V"]),
             ADT=torch.empty(B, H, L, **f32), DT=torch.empty(B, H, L, **f32),
             Trap=torch.empty(B, H, L, **f32), Q_bias=torch.empty(H, N, **f32),
             K_bias=torch.empty(H, N, **f32), Angles=torch.empty(B, L, H, R, **f32),
             D=None if p["D"] is None else torch.empty(H, **f32),
             Z=None if p["Z"] is None else torch.empty_like(p["Z"]))
    if B and L:
        lib = _lib.load()
        if saved is None:
            ws_bytes = lib.m3_chunk_scan_bwd_ws_bytes(B, L, H, HQ, N, P, R, int(chunk_size), io)
        else:
            ws_bytes = lib.m3_chunk_scan_bwd_saved_ws_bytes(B, L, H, HQ, N, P, R, int(chunk_size), io)
        if ws_bytes == 0:
            raise _lib.Mamba3LibraryError(
                f"no backward kernel for dtype={dt} d_state={N} headdim={P} rope angles={R}")
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        ptrs = (_ptr(p["Q"]), _ptr(p["K"]), _ptr(p["V"]), _ptr(p["ADT"]), _ptr(p["DT"]), _ptr(p["Trap"]),
                _ptr(p["Q_bias"]), _ptr(p["K_bias"]), _ptr(p["Angles"]), _ptr(p["D"]), _ptr(p["Z"]), _ptr(dO),
                _ptr(g["Q"]), _ptr(g["K"]), _ptr(g["V"]), _ptr(g["ADT"]), _ptr(g["DT"]), _ptr(g["Trap"]),
                _ptr(g["Q_bias"]), _ptr(g["K_bias"]), _ptr(g["Angles"]), _ptr(g["D"]), _ptr(g["Z"]),
                B, L, H, HQ, N, P, R, int(chunk_size), io)
        if saved is None:
            rc = lib.m3_chunk_scan_bwd(*ptrs, ws.data_ptr(), ws_bytes, _stream(p["V"]))
        else:
            rc = lib.m3_chunk_scan_bwd_saved(*ptrs, saved.data_ptr(), saved.numel(), ws.data_ptr(), ws_bytes,
                                             _stream(p["V"]))
        _lib.check(rc, "m3_chunk_scan_bwd")
    else:
        for t in g.values():
            if t is not None:
                t.zero_()
    order = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")
    if unbatched:
        return tuple(None if g[k] is None else (g[k] if k in ("Q_bias", "K_bias", "D") else g[k][0])
                     for k in order)
    return tuple(g[k] for k in order)


def mamba3_siso_hip_fwd_train(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D=None, Z=None,
                              chunk_size: int = 64, seq_split: bool = True):
    """The reference's mamba3_siso_fwd (mamba3_ops.py:788-818): the output and the
    residuals for mamba3_siso_hip_bwd(..., saved=...) (None where the shape has no
    saved-state path)."""
    return _forward_train((Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z), chunk_size, seq_split)


class _Mamba3Siso(torch.autograd.Function):
    """mamba3_siso_hip with its backward: the reference's custom_vjp pair
    (mamba3_ops.py:909-1045).  Saves the inputs and the forward's chunk states, which
    the backward reads instead of recomputing them."""

    @staticmethod
    def forward(ctx, chunk_size, seq_split, *args):
        ctx.chunk_size = chunk_size
        out, saved = _forward_train(args, chunk_size, seq_split)
        ctx.save_for_backward(*(t if isinstance(t, torch.Tensor) else None for t in args), saved)
        return out

    @staticmethod
    def backward(ctx, dout):
        *args, saved = ctx.saved_tensors
        grads = mamba3_siso_hip_bwd(*args, dout, chunk_size=ctx.chunk_size, saved=saved)
        out = []
        for t, gr in zip(args, grads):
            out.append(None if t is None or gr is None else gr.to(t.dtype))
        return (None, None, *out)


def mamba3_ssd_chunked_hip(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z,
                           chunk_size: int = 64) -> torch.Tensor:
    """The oracle's signature (mamba3_jax.py:327-331): angles 7th, D and Z required
    there (None accepted here).  Same computation as mamba3_siso_hip."""
    return mamba3_siso_hip(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, angles, D, Z, chunk_size)


def new_carry(B: int, H: int, N: int, P: int, R: int, device) -> Tuple[torch.Tensor, ...]:
    """Zero recurrent carry (theta (B,H,R), ssm (B,H,P,N), k (B,H,N), v (B,H,P)), the
    layout of the reference's Mamba3 decode carry (layers.py:243-256 without the
    singleton dims)."""
    z = dict(device=device, dtype=torch.float32)
    return (torch.zeros(B, H, R, **z), torch.zeros(B, H, P, N, **z),
            torch.zeros(B, H, N, **z), torch.zeros(B, H, P, **z))


def mamba3_siso_hip_carry(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D=None, Z=None,
                          chunk_size: int = 64, initial_carry=None, seq_split: bool = True):
    """Prefill that also consumes and returns the recurrent carry, so decode can
    continue where prefill stopped (the Triton kernel's HAS_INITIAL_STATES /
    RETURN_FINAL_STATES, siso_fwd.py:76-77).  Batched inputs only.
    Returns (Out, (theta, ssm, k, v))."""
    p, dims, unbatched = _prep(Q, K, V, ADT, DT, Trap, Q_bias, K_bias, Angles, D, Z)
    _req(not unbatched, "mamba3_siso_hip_carry takes batched (B, L, ...) inputs")
    B, L, H, HQ, N, P, R = dims
    out = torch.empty_like(p["V"])
    fin = new_carry(B, H, N, P, R, p["V"].device)
    init = None
    if initial_carry is not None:
        init = tuple(_f32(t) for t in initial_carry)
        shapes = [(B, H, R), (B, H, P, N), (B, H, N), (B, H, P)]
        for t, s, n in zip(init, shapes, ("theta", "ssm", "k", "v")):
            _req(tuple(t.shape) == s, f"initial carry {n} must be {s}, got {tuple(t.shape)}")
    if out.numel():
        _launch(p, dims, chunk_size, out, init=init, fin=fin, seq_split=seq_split)
    elif init is not None:
        fin = tuple(t.clone() for t in init)
    return out, fin


# ----------------------------------------------------------------- shared B/C
def _prep_shared(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z, cdt=None):
    """Validate and normalise the fused path's layout: Q, K (B, L, N) and angle
    rates (B, L, R), shared over the H heads of V (B, L, H, P); Q, K, V and Z in
    the compute dtype cdt (default: pallas_compute_dtype of V's dtype)."""
    mamba3_contraction_precision_mode()
    unbatched = V.dim() == 3
    if unbatched:
        Q, K, V, ADT, DT, Trap, angles = Q[None], K[None], V[None], ADT[None], DT[None], Trap[None], angles[None]
        if Z is not None and Z.dim() == 3:
            Z = Z[None]
    if angles.dim() == 4:
        angles = angles[:, :, 0]
    _req(Q.dim() == 3 and tuple(Q.shape) == tuple(K.shape),
         "the fused path takes Q and K as (L, d_state), shared over heads")
    B, L, N = Q.shape
    _req(V.dim() == 4 and tuple(V.shape[:2]) == (B, L), f"V must be {(B, L, '<H>', '<P>')}, got {tuple(V.shape)}")
    H, P = V.shape[2], V.shape[3]
    for name, t in (("Q", Q), ("K", K), ("V", V)):
        _dev(t, name)
    for name, t in (("ADT", ADT), ("DT", DT), ("Trap", Trap)):
        _req(tuple(t.shape) == (B, H, L), f"{name} must be {(B, H, L)}, got {tuple(t.shape)}")
    for name, t in (("Q_bias", Q_bias), ("K_bias", K_bias)):
        _req(tuple(t.shape) == (H, N), f"{name} must be {(H, N)}, got {tuple(t.shape)}")
    _req(angles.dim() == 3 and tuple(angles.shape[:2]) == (B, L),
         f"angles must be (L, R) or (L, 1, R), got {tuple(angles.shape)}")
    R = angles.shape[-1]
    _req(R <= N // 2, f"headdim_angles ({R}) must be <= headdim_qk // 2 ({N // 2})")
    if D is not None:
        _req(tuple(D.shape) == (H,), f"D must be {(H,)}, got {tuple(D.shape)}")
    if Z is not None:
        _req(tuple(Z.shape) == (B, L, H, P), f"Z must be {(B, L, H, P)}, got {tuple(Z.shape)}")
    _req(V.dtype in _IO, f"V dtype must be float32 or bfloat16, got {V.dtype}")
    dt = cdt or pallas_compute_dtype(V.dtype)
    p = dict(Q=Q.to(dt).contiguous(), K=K.to(dt).contiguous(), V=V.to(dt).contiguous(), ADT=_f32(ADT), DT=_f32(DT),
             Trap=_f32(Trap), Q_bias=_f32(Q_bias), K_bias=_f32(K_bias), Angles=_f32(angles),
             D=None if D is None else _f32(D), Z=None if Z is None else Z.to(dt).contiguous())
    return p, (B, L, H, N, P, R), unbatched


def _shared_forward(args, chunk_size, seq_split, train=False, cdt=None):
    """The fused path's forward; with ``train`` also the residuals of its backward
    (None where the shape has no saved-state path).  Returns (out, saved), out in V's
    dtype."""
    p, (B, L, H, N, P, R), unbatched = _prep_shared(*args, cdt=cdt)
    out = torch.empty_like(p["V"])
    saved = None
    if out.numel():
        lib = _lib.load()
        io = _IO[p["V"].dtype]
        ws_bytes = lib.m3_chunk_scan_ws_bytes(B, L, H, N, P, R, int(chunk_size), io) if seq_split else 0
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=p["V"].device)
        common = (_ptr(p["Q"]), _ptr(p["K"]), _ptr(p["V"]), _ptr(p["ADT"]), _ptr(p["DT"]), _ptr(p["Trap"]),
                  _ptr(p["Q_bias"]), _ptr(p["K_bias"]), _ptr(p["Angles"]), _ptr(p["D"]), _ptr(p["Z"]), _ptr(out),
                  B, L, H, N, P, R, int(chunk_size), io)
        nbytes = lib.m3_chunk_scan_saved_bytes(B, L, H, N, P, R, io) if train else 0
        kbwd = 64 if io == _lib.DTYPE_BF16 else 32
        if nbytes and int(chunk_size) % kbwd == 0 and \
                lib.m3_chunk_scan_impl(io, N, P, R, int(chunk_size)) == _lib.IMPL_CHUNKED_MFMA:
            saved = torch.empty(nbytes, dtype=torch.uint8, device=p["V"].device)
            rc = lib.m3_chunk_scan_fwd_train_shared(*common, saved.data_ptr(), nbytes,
                                                    ws.data_ptr() if ws_bytes else None, ws_bytes, _stream(p["V"]))
            _lib.check(rc, "m3_chunk_scan_fwd_train_shared")
        else:
            rc = lib.m3_chunk_scan_fwd_shared(*common, ws.data_ptr() if ws_bytes else None, ws_bytes,
                                              _stream(p["V"]))
            _lib.check(rc, "m3_chunk_scan_fwd_shared")
    out = out.to(args[2].dtype)
    return (out[0] if unbatched else out), saved


def mamba3_ssd_chunked_shared_hip_fwd_train(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D=None, Z=None,
                                            chunk_size: int = 64, seq_split: bool = True, compute_dtype=None):
    """The fused path's forward with the residuals its backward reads (the state and
    rope angle entering every chunk and, float32, the output before the gate), as
    the reference's fused chunk scan saves them (chunk_scan_fwd_rule,
    mamba3_pallas.py:602-604).  Returns (out, saved); saved is None where the shape
    has no saved-state path."""
    return _shared_forward((Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z), chunk_size, seq_split,
                           train=True, cdt=compute_dtype)


def mamba3_ssd_chunked_shared_hip_bwd(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z, dOut,
                                      chunk_size: int = 64, saved: Optional[torch.Tensor] = None,
                                      compute_dtype=None):
    """All eleven input gradients of mamba3_ssd_chunked_shared_hip, in its argument
    order (Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z); dQ, dK and dangles
    are summed over heads (shaped like the shared inputs); dD, dZ None when absent.
    dQ, dK, dV and dZ come in the compute dtype.  ``saved``: the residuals of
    mamba3_ssd_chunked_shared_hip_fwd_train on the same inputs (with the same compute
    dtype); without them the chunk states are recomputed."""
    ang_in = angles
    p, (B, L, H, N, P, R), unbatched = _prep_shared(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z,
                                                    cdt=compute_dtype)
    io = _IO[p["V"].dtype]
    dO = (dOut[None] if unbatched else dOut).to(p["V"].dtype).contiguous()
    _req(tuple(dO.shape) == (B, L, H, P), f"dOut must be {(B, L, H, P)}, got {tuple(dOut.shape)}")
    dev = p["V"].device
    f32 = dict(device=dev, dtype=torch.float32)
    g = dict(Q=torch.empty_like(p["Q"]), K=torch.empty_like(p["K"]), V=torch.empty_like(p["V"]),
             ADT=torch.empty(B, H, L, **f32), DT=torch.empty(B, H, L, **f32), Trap=torch.empty(B, H, L, **f32),
             Angles=torch.empty(B, L, R, **f32), Q_bias=torch.empty(H, N, **f32), K_bias=torch.empty(H, N, **f32),
             D=None if p["D"] is None else torch.empty(H, **f32),
             Z=None if p["Z"] is None else torch.empty_like(p["Z"]))
    if B and L:
        lib = _lib.load()
        if saved is None:
            ws_bytes = lib.m3_chunk_scan_bwd_shared_ws_bytes(B, L, H, N, P, R, int(chunk_size), io)
        else:
            ws_bytes = lib.m3_chunk_scan_bwd_saved_shared_ws_bytes(B, L, H, N, P, R, int(chunk_size), io)
        if ws_bytes == 0:
            raise _lib.Mamba3LibraryError(
                f"no backward kernel for dtype={p['V'].dtype} d_state={N} headdim={P} rope angles={R}")
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        ptrs = (_ptr(p["Q"]), _ptr(p["K"]), _ptr(p["V"]), _ptr(p["ADT"]), _ptr(p["DT"]), _ptr(p["Trap"]),
                _ptr(p["Q_bias"]), _ptr(p["K_bias"]), _ptr(p["Angles"]), _ptr(p["D"]), _ptr(p["Z"]), _ptr(dO),
                _ptr(g["Q"]), _ptr(g["K"]), _ptr(g["V"]), _ptr(g["ADT"]), _ptr(g["DT"]), _ptr(g["Trap"]),
                _ptr(g["Q_bias"]), _ptr(g["K_bias"]), _ptr(g["Angles"]), _ptr(g["D"]), _ptr(g["Z"]),
                B, L, H, N, P, R, int(chunk_size), io)
        if saved is None:
            rc = lib.m3_chunk_scan_bwd_shared(*ptrs, ws.data_ptr(), ws_bytes, _stream(p["V"]))
        else:
            rc = lib.m3_chunk_scan_bwd_saved_shared(*ptrs, saved.data_ptr(), saved.numel(), ws.data_ptr(),
                                                    ws_bytes, _stream(p["V"]))
        _lib.check(rc, "m3_chunk_scan_bwd_shared")
    else:
        for t in g.values():
            if t is not None:
                t.zero_()
    dang = g["Angles"].reshape(ang_in.shape if not unbatched else (1,) + tuple(ang_in.shape))
    out = dict(g, Angles=dang)
    order = ("Q", "K", "V", "ADT", "DT", "Trap", "Angles", "Q_bias", "K_bias", "D", "Z")
    if unbatched:
        return tuple(None if out[k] is None else (out[k] if k in ("Q_bias", "K_bias", "D") else out[k][0])
                     for k in order)
    return tuple(out[k] for k in order)


class _Mamba3Shared(torch.autograd.Function):
    """mamba3_ssd_chunked_shared_hip with its backward (the fused path is
    differentiable, mamba3_pallas.py:824-830).  As the reference's fused chunk scan
    (chunk_scan_fwd_rule / chunk_scan_bwd_rule, mamba3_pallas.py:602-645), the
    forward saves the states entering every chunk, which the backward reads instead
    of recomputing them."""

    @staticmethod
    def forward(ctx, chunk_size, seq_split, cdt, *args):
        ctx.chunk_size, ctx.cdt = chunk_size, cdt
        out, saved = _shared_forward(args, chunk_size, seq_split, train=True, cdt=cdt)
        ctx.save_for_backward(*(t if isinstance(t, torch.Tensor) else None for t in args), saved)
        return out

    @staticmethod
    def backward(ctx, dout):
        *args, saved = ctx.saved_tensors
        grads = mamba3_ssd_chunked_shared_hip_bwd(*args, dout, chunk_size=ctx.chunk_size, saved=saved,
                                                  compute_dtype=ctx.cdt)
        return (None, None, None,
                *(None if t is None or gr is None else gr.to(t.dtype) for t, gr in zip(args, grads)))


def mamba3_ssd_chunked_shared_hip(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D=None, Z=None,
                                  chunk_size: int = 64, seq_split: bool = True,
                                  compute_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """The reference's fused-path entry with B and C shared over heads,
    mamba3_ssd_chunked_pallas(Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z,
    chunk_size) (src/base_model/models/mamba3_pallas.py:813-849): Q, K (L, N) shared
    over heads; angles (L, R), (L, 1, R) or (L, nh, R); V, Z (L, nh, P); ADT, DT, Trap
    (nh, L); Q_bias, K_bias (nh, N); D (nh,); optionally a leading batch dim on
    every per-sequence input.  Same result as the per-head scan with Q, K and angles
    repeated over heads.  Differentiable (torch autograd).

    ``compute_dtype``: the MFMA operand dtype (the reference's compute_dtype,
    mamba3_pallas.py:817-839); None reads MAMBA3_PALLAS_DTYPE, then V's dtype
    (pallas_compute_dtype).  Q, K, V and Z are cast to it; the output comes back in
    V's dtype."""
    cdt = compute_dtype or pallas_compute_dtype(V.dtype)
    _req(cdt in _IO, f"compute_dtype must be float32 or bfloat16, got {cdt}")
    per_head = angles.dim() == (4 if V.dim() == 4 else 3) and angles.shape[-2] > 1
    if per_head:
        # angle rates per head: the per-head path with one shared Q/K head (Hqk = 1)
        Zc = None if Z is None else Z.to(cdt)
        out = mamba3_siso_hip(Q.unsqueeze(-2).to(cdt), K.unsqueeze(-2).to(cdt), V.to(cdt), ADT, DT, Trap,
                              Q_bias, K_bias, angles, D, Zc, chunk_size=chunk_size, seq_split=seq_split)
        return out.to(V.dtype)
    args = (Q, K, V, ADT, DT, Trap, angles, Q_bias, K_bias, D, Z)
    if torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in args):
        return _Mamba3Shared.apply(int(chunk_size), bool(seq_split), cdt, *args)
    return _shared_forward(args, chunk_size, seq_split, cdt=cdt)[0]
