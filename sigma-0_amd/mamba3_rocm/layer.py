"""The Mamba3 mixer layer on gfx950: Mamba3SSM's forward
(src/base_model/models/mamba3.py:191-331, the fused path with B and C shared over
heads).

    proj = x @ in_proj                      library GEMM in the compute dtype
    m3_layer_pre                            BCNorm, decay, trapezoid, rates
    m3_layer_scan                           the scan, x and z read in place from proj
    m3_layer_post                           output RMSNorm
    out = ... @ out_proj                    library GEMM

Where the projection rows are not a multiple of 16 bytes, m3_layer_pre also copies
x and z out of proj and the scan is m3_chunk_scan_fwd_shared on the copies.

``Mamba3Layer.train_forward`` is the same forward made differentiable (gradients for
x and for every parameter, as autodiff of Mamba3SSM gives them).  Its scan is the
training pair, which saves the states entering every chunk for the backward instead
of recomputing them: m3_layer_scan_train (x and z read in place) and
m3_layer_scan_bwd, which writes dV and dZ straight into the x and z columns of the
in_proj output's gradient; where the rows do not allow that, m3_layer_pre copies x
and z and the pair is m3_chunk_scan_fwd_train_shared / m3_chunk_scan_bwd_saved_shared.
The backward is the library GEMMs' gradients, m3_layer_post_bwd (the output RMSNorm),
the scan's backward and m3_layer_pre_bwd (BCNorm, the decay's chain rule with the
A_floor clip, trap and angles, written into the in_proj output's gradient).

Parameters keep the reference's names and layouts (flax Dense kernels are
(in, out)) and stay float32; ``dtype`` is the compute dtype of the projections
and the scan's operands (the reference's ``dtype`` field, mamba3.py:103-110).
"""
from __future__ import annotations

import math
from typing import Dict

import torch

from . import _lib
from .ops import (_IO, _ptr, _stream, mamba3_siso_hip_carry, mamba3_ssd_chunked_shared_hip,
                  mamba3_ssd_chunked_shared_hip_bwd, mamba3_ssd_chunked_shared_hip_fwd_train, new_carry,
                  pallas_compute_dtype)

PARAM_NAMES = ("in_proj", "dt_bias", "B_bias", "C_bias", "B_norm", "C_norm", "D", "out_norm", "out_proj")


class Mamba3Layer:
    """Forward of one Mamba3SSM layer (d_model -> d_model) on a ROCm device."""

    def __init__(self, params: Dict[str, torch.Tensor], d_model: int, d_state: int = 128, expand: int = 2,
                 headdim: int = 64, chunk_size: int = 64, rope_fraction: float = 0.5, A_floor: float = 1e-4,
                 dtype: torch.dtype = torch.bfloat16, eps: float = 1e-6):
        d_inner_target = expand * d_model
        self.hd = min(headdim, d_inner_target)
        self.nh = max(1, d_inner_target // self.hd)
        split = int(d_state * rope_fraction)
        split -= split % 2
        self.R = split // 2
        self.N, self.d_model, self.chunk_size = d_state, d_model, chunk_size
        self.A_floor, self.eps, self.dtype = float(A_floor), float(eps), dtype
        self.d_inner = self.nh * self.hd
        self.d_in_proj = 2 * self.d_inner + 2 * d_state + 3 * self.nh + self.R
        if dtype not in _IO:
            raise ValueError(f"dtype must be float32 or bfloat16, got {dtype}")
        p = {k: params[k] for k in PARAM_NAMES}
        if not p["in_proj"].is_cuda:
            raise ValueError("Mamba3Layer parameters must be ROCm device tensors (no CPU path)")
        expect = dict(in_proj=(d_model, self.d_in_proj), dt_bias=(self.nh,), B_bias=(self.nh, d_state),
                      C_bias=(self.nh, d_state), B_norm=(d_state,), C_norm=(d_state,), D=(self.nh,),
                      out_norm=(self.d_inner,), out_proj=(self.d_inner, d_model))
        for k, shape in expect.items():
            if tuple(p[k].shape) != shape:
                raise ValueError(f"{k} must be {shape}, got {tuple(p[k].shape)}")
        self.params = {k: v.to(torch.float32).contiguous() for k, v in p.items()}
        # the projections' operands in the compute dtype (nn.Dense(dtype=...) casts them)
        self.w_in = self.params["in_proj"].to(dtype).contiguous()
        self.w_out = self.params["out_proj"].to(dtype).contiguous()
        # "in_place" or "copies", prefixed "train_" for train_forward (the scan's training
        # forward): how the last forward fed x and z to the scan
        self.last_scan = None
        self.last_compute_dtype = None   # the scan's operand dtype in the last forward

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x (B, L, d_model) or (L, d_model) -> the same shape, in the compute dtype."""
        return self._run(x, self.w_in, self.w_out)[0]

    def new_carry(self, batch: int, device=None):
        """The zero recurrent carry of ``batch`` sequences: theta (B, H, R), ssm (B, H, P,
        N), k (B, H, N), v (B, H, P), float32 (the reference's decode carry,
        layers.py:243-256, without its singleton dims)."""
        return new_carry(batch, self.nh, self.N, self.hd, self.R, device or self.w_in.device)

    def prefill(self, x: torch.Tensor, carry=None):
        """The forward on x (B, L, d_model) that also continues from a carry (or from
        zero) and returns the carry after the last token, so that step() or another
        prefill continues the sequences.  Returns (out, carry)."""
        out, _, fin = self._run(x, self.w_in, self.w_out, init=carry, want_carry=True)
        return out, fin

    def step(self, x_t: torch.Tensor, carry):
        """One token per sequence, as Mamba3SSM.__call_rnn__ runs it (mamba3.py:466-568):
        x_t (B, d_model) -> (out (B, d_model) in the compute dtype, carry), the carry
        updated in place.  The in_proj GEMM, m3_layer_decode_step (m3_layer_pre's work on
        the token and the decode update in one launch: B and C shared over heads, trap
        through the sigmoid as the reference's recurrent path applies it),
        m3_layer_post and the out_proj GEMM."""
        from .decode import recurrent_angle_mode, recurrent_diagonal_mode
        from .ops import mamba3_contraction_precision_mode
        Bn = x_t.shape[0]
        dt, dev = self.dtype, x_t.device
        nh, hd, N, R = self.nh, self.hd, self.N, self.R
        lib, io, pp = _lib.load(), _IO[dt], self.params
        theta, ssm, kprev, vprev = carry
        for name, t, shape in (("theta", theta, (Bn, nh, R)), ("ssm", ssm, (Bn, nh, hd, N)),
                               ("k", kprev, (Bn, nh, N)), ("v", vprev, (Bn, nh, hd))):
            if not (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() and tuple(t.shape) == shape):
                raise ValueError(f"carry {name} must be a contiguous float32 device tensor of shape {shape} "
                                 "(it is updated in place)")
        mamba3_contraction_precision_mode()     # the reference's decode reads it too (mamba3.py:545)
        angle, diag = recurrent_angle_mode(), recurrent_diagonal_mode()
        proj = torch.matmul(x_t.to(dt).reshape(Bn, 1, self.d_model), self.w_in).contiguous()
        y = torch.empty(Bn, 1, self.d_inner, device=dev, dtype=dt)
        _lib.check(lib.m3_layer_decode_step(
            _ptr(proj), _ptr(pp["dt_bias"]), _ptr(pp["B_norm"]), _ptr(pp["C_norm"]), _ptr(pp["B_bias"]),
            _ptr(pp["C_bias"]), _ptr(pp["D"]), _ptr(theta), _ptr(ssm), _ptr(kprev), _ptr(vprev), _ptr(y),
            Bn, nh, hd, N, R, self.A_floor, self.eps, io, 1 if angle == "wrapped" else 0,
            1 if diag == "legacy_double" else 0, _stream(proj)), "m3_layer_decode_step")
        yn = torch.empty(Bn, 1, self.d_inner, device=dev, dtype=dt)
        _lib.check(lib.m3_layer_post(_ptr(y), _ptr(pp["out_norm"]), _ptr(yn), Bn, 1, self.d_inner, self.eps, io,
                                     _stream(y)), "m3_layer_post")
        return torch.matmul(yn, self.w_out).reshape(Bn, self.d_model), carry

    def train_forward(self, x: torch.Tensor) -> torch.Tensor:
        """forward, differentiable: gradients flow to x and to the parameter tensors the
        layer was built with (``self.params``, float32; those with requires_grad get
        theirs).  The compute-dtype copies of the projection kernels are taken from the
        parameters at every call, so updates in place are seen."""
        return _LayerTrain.apply(self, x, *(self.params[k] for k in PARAM_NAMES))

    def _run(self, x: torch.Tensor, w_in: torch.Tensor, w_out: torch.Tensor, keep: bool = False, init=None,
             want_carry: bool = False):
        """The forward; with ``keep`` (train_forward) also the intermediates the backward
        reads, the scan's residuals among them; with ``want_carry`` the scan continues
        from ``init`` (or zero) and the carry after the last token is returned.
        Returns (out, saved, carry)."""
        if keep and want_carry:
            raise ValueError("the training forward takes no carry")
        unbatched = x.dim() == 2
        if unbatched:
            x = x[None]
        B, L, _ = x.shape
        dt, dev = self.dtype, x.device
        nh, hd, N, R = self.nh, self.hd, self.N, self.R
        xin = x.to(dt)
        proj = torch.matmul(xin, w_in).contiguous()                  # (B, L, d_in_proj)
        Q = torch.empty(B, L, N, device=dev, dtype=dt)
        K = torch.empty_like(Q)
        f32 = dict(device=dev, dtype=torch.float32)
        ADT, DT, Trap = (torch.empty(B, nh, L, **f32) for _ in range(3))
        Ang = torch.empty(B, L, R, **f32)
        lib = _lib.load()
        io = _IO[dt]
        pp = self.params
        st = _stream(proj)

        def pre(V, Z):
            _lib.check(lib.m3_layer_pre(_ptr(proj), _ptr(pp["dt_bias"]), _ptr(pp["B_norm"]), _ptr(pp["C_norm"]),
                                        _ptr(Q), _ptr(K), _ptr(V), _ptr(Z), _ptr(ADT), _ptr(DT), _ptr(Trap),
                                        _ptr(Ang), B, L, nh, hd, N, R, self.A_floor, self.eps, io, st),
                       "m3_layer_pre")

        # Q = C, K = B (_forward_pallas, mamba3.py:413-425).  x and z are read in place
        # from proj when its rows and the x block are 16-byte aligned and the shape has
        # the chunked kernel (m3_layer_scan's conditions); otherwise they are copied.
        # MAMBA3_PALLAS_DTYPE may ask for scan operands in another dtype than the
        # layer's (mamba3_pallas.py:112-122, 838-839): then the copies are cast to it.
        cdt = pallas_compute_dtype(dt)
        es = proj.element_size()
        in_place = (cdt == dt and (self.d_in_proj * es) % 16 == 0 and (self.d_inner * es) % 16 == 0
                    and proj.data_ptr() % 16 == 0
                    and lib.m3_chunk_scan_impl(io, N, hd, R, self.chunk_size) == _lib.IMPL_CHUNKED_MFMA)
        carry = None
        if want_carry:
            if init is not None:
                init = tuple(t.to(torch.float32).contiguous() for t in init)
                shapes = [(B, nh, R), (B, nh, hd, N), (B, nh, N), (B, nh, hd)]
                for t, s_, n in zip(init, shapes, ("theta", "ssm", "k", "v")):
                    if tuple(t.shape) != s_:
                        raise ValueError(f"carry {n} must be {s_}, got {tuple(t.shape)}")
            carry = new_carry(B, nh, N, hd, R, dev)
        sbytes = 0
        if keep and in_place:
            # in place in training: the saved-state pair must exist for the shape (a
            # backward kernel, and the forward's chunk a multiple of the backward's)
            kbwd = 64 if io == _lib.DTYPE_BF16 else 32
            if (self.chunk_size % kbwd == 0
                    and lib.m3_chunk_scan_bwd_saved_shared_ws_bytes(B, L, nh, N, hd, R, self.chunk_size, io)):
                sbytes = lib.m3_chunk_scan_saved_bytes(B, L, nh, N, hd, R, io)
            in_place = sbytes > 0
        self.last_scan = ("train_" if keep else "") + ("in_place" if in_place else "copies")
        self.last_compute_dtype = cdt
        V = Z = scan_saved = None
        if in_place:
            pre(None, None)
            y = torch.empty(B, L, nh, hd, device=dev, dtype=dt)
            ws_bytes = lib.m3_chunk_scan_ws_bytes(B, L, nh, N, hd, R, self.chunk_size, io)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
            args = (_ptr(Q), _ptr(K), _ptr(proj), self.d_in_proj, _ptr(ADT), _ptr(DT), _ptr(Trap), _ptr(Ang),
                    _ptr(pp["C_bias"]), _ptr(pp["B_bias"]), _ptr(pp["D"]), _ptr(y), B, L, nh, N, hd, R,
                    self.chunk_size, io)
            wsa = (ws.data_ptr() if ws_bytes else None, ws_bytes, st)
            if keep:
                scan_saved = torch.empty(sbytes, dtype=torch.uint8, device=dev)
                _lib.check(lib.m3_layer_scan_train(*args, scan_saved.data_ptr(), sbytes, *wsa), "m3_layer_scan_train")
            elif want_carry:
                cin = tuple(_ptr(t) for t in init) if init is not None else (None,) * 4
                _lib.check(lib.m3_layer_scan_carry(*args[:12], *cin, *(_ptr(t) for t in carry), *args[12:], *wsa),
                           "m3_layer_scan_carry")
            else:
                _lib.check(lib.m3_layer_scan(*args, *wsa), "m3_layer_scan")
        else:
            V = torch.empty(B, L, nh, hd, device=dev, dtype=dt)
            Z = torch.empty_like(V)
            pre(V, Z)
            scan_args = (Q, K, V, ADT, DT, Trap, Ang, pp["C_bias"], pp["B_bias"], pp["D"], Z)
            if keep:
                y, scan_saved = mamba3_ssd_chunked_shared_hip_fwd_train(*scan_args, chunk_size=self.chunk_size,
                                                                        compute_dtype=cdt)
            elif want_carry:
                # the per-head carry contract with one Q/K head shared by all and the
                # shared angle rates repeated over the heads
                c = lambda t: t.to(cdt)  # noqa: E731
                y, carry = mamba3_siso_hip_carry(c(Q)[:, :, None], c(K)[:, :, None], c(V), ADT, DT, Trap,
                                                 pp["C_bias"], pp["B_bias"], Ang[:, :, None].expand(B, L, nh, R),
                                                 pp["D"], c(Z), chunk_size=self.chunk_size, initial_carry=init)
                y = y.to(dt)
            else:
                y = mamba3_ssd_chunked_shared_hip(*scan_args, chunk_size=self.chunk_size, compute_dtype=cdt)
        yn = torch.empty(B, L, self.d_inner, device=dev, dtype=dt)
        _lib.check(lib.m3_layer_post(_ptr(y), _ptr(pp["out_norm"]), _ptr(yn), B, L, self.d_inner, self.eps, io,
                                     _stream(y)), "m3_layer_post")
        out = torch.matmul(yn, w_out)
        saved = (dict(xin=xin, proj=proj, Q=Q, K=K, V=V, Z=Z, ADT=ADT, DT=DT, Trap=Trap, Ang=Ang, y=y, yn=yn,
                      cdt=cdt, scan=scan_saved, in_place=in_place) if keep else None)
        return (out[0] if unbatched else out), saved, carry

    def _backward(self, saved, dout: torch.Tensor, w_in: torch.Tensor, w_out: torch.Tensor):
        """Gradients of x and of the parameters (PARAM_NAMES order, float32) from the
        output cotangent, as autodiff of Mamba3SSM.__call__ (mamba3.py:191-331) gives
        them: the GEMMs' gradients (library GEMMs in the compute dtype, as the
        reference's bf16 layer differentiates its bf16 dots), m3_layer_post_bwd, the
        shared scan's backward and m3_layer_pre_bwd; the roundings of the compute
        dtype pass gradients through unchanged."""
        xin, proj, y, yn = saved["xin"], saved["proj"], saved["y"], saved["yn"]
        B, L, _ = xin.shape
        dt, dev = self.dtype, xin.device
        nh, hd, N, R, di, eps = self.nh, self.hd, self.N, self.R, self.d_inner, self.eps
        pp = self.params
        lib = _lib.load()
        io = _IO[dt]
        f32 = dict(device=dev, dtype=torch.float32)
        d_out = dout.reshape(B, L, self.d_model).to(dt).contiguous()
        # out = (y rsqrt(mean y^2 + eps) out_norm) @ out_proj  (_post_norm_and_project, :281-331)
        g_out_proj = (yn.reshape(-1, di).t() @ d_out.reshape(-1, self.d_model)).float()
        d_yn = torch.matmul(d_out, w_out.t()).contiguous()
        d_y = torch.empty_like(d_yn)
        g_out_norm = torch.empty(di, **f32)
        ws = torch.empty(max(lib.m3_layer_post_bwd_ws_bytes(B, L, di), 16), dtype=torch.uint8, device=dev)
        _lib.check(lib.m3_layer_post_bwd(_ptr(y), _ptr(d_yn), _ptr(pp["out_norm"]), _ptr(d_y), _ptr(g_out_norm), B, L,
                                         di, eps, io, ws.data_ptr(), ws.numel(), _stream(y)), "m3_layer_post_bwd")
        # the scan (Q = C, K = B shared over heads), from the training forward's residuals
        # (recomputed where the shape has none)
        d_proj = torch.empty_like(proj)
        if saved["in_place"]:
            # dV and dZ straight into d_proj's x and z columns
            dC, dB = torch.empty_like(saved["Q"]), torch.empty_like(saved["K"])
            dADT, dDT, dTrap = (torch.empty(B, nh, L, **f32) for _ in range(3))
            dAng = torch.empty(B, L, R, **f32)
            g_C_bias, g_B_bias, g_D = torch.empty(nh, N, **f32), torch.empty(nh, N, **f32), torch.empty(nh, **f32)
            sb = saved["scan"]
            wsb = lib.m3_chunk_scan_bwd_saved_shared_ws_bytes(B, L, nh, N, hd, R, self.chunk_size, io)
            ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
            _lib.check(lib.m3_layer_scan_bwd(
                _ptr(saved["Q"]), _ptr(saved["K"]), _ptr(proj), self.d_in_proj, _ptr(saved["ADT"]), _ptr(saved["DT"]),
                _ptr(saved["Trap"]), _ptr(saved["Ang"]), _ptr(pp["C_bias"]), _ptr(pp["B_bias"]), _ptr(pp["D"]),
                _ptr(d_y), _ptr(dC), _ptr(dB), _ptr(d_proj), _ptr(dADT), _ptr(dDT), _ptr(dTrap), _ptr(g_C_bias),
                _ptr(g_B_bias), _ptr(dAng), _ptr(g_D), B, L, nh, N, hd, R, self.chunk_size, io, sb.data_ptr(),
                sb.numel(), ws.data_ptr(), wsb, _stream(proj)), "m3_layer_scan_bwd")
            dV = dZ = None
        else:
            g = mamba3_ssd_chunked_shared_hip_bwd(saved["Q"], saved["K"], saved["V"], saved["ADT"], saved["DT"],
                                                  saved["Trap"], saved["Ang"], pp["C_bias"], pp["B_bias"], pp["D"],
                                                  saved["Z"], d_y.reshape(B, L, nh, hd), chunk_size=self.chunk_size,
                                                  saved=saved["scan"], compute_dtype=saved["cdt"])
            dC, dB, dV, dADT, dDT, dTrap, dAng, g_C_bias, g_B_bias, g_D, dZ = g
            c = lambda t: t.to(dt).contiguous()  # noqa: E731
            dC, dB, dV, dZ = c(dC), c(dB), c(dV), c(dZ)
        # _preprocess (:203-268): BCNorm, the decay, trap and angles back to the in_proj output
        g_dt_bias, g_B_norm, g_C_norm = torch.empty(nh, **f32), torch.empty(N, **f32), torch.empty(N, **f32)
        ws = torch.empty(max(lib.m3_layer_pre_bwd_ws_bytes(B, L, nh, N), 16), dtype=torch.uint8, device=dev)
        _lib.check(lib.m3_layer_pre_bwd(_ptr(proj), _ptr(pp["dt_bias"]), _ptr(pp["B_norm"]), _ptr(pp["C_norm"]),
                                        _ptr(dC), _ptr(dB), _ptr(dV), _ptr(dZ), _ptr(dADT), _ptr(dDT), _ptr(dTrap),
                                        _ptr(dAng), _ptr(d_proj), _ptr(g_dt_bias), _ptr(g_B_norm), _ptr(g_C_norm),
                                        B, L, nh, hd, N, R, self.A_floor, eps, io, ws.data_ptr(), ws.numel(),
                                        _stream(proj)), "m3_layer_pre_bwd")
        g_in_proj = (xin.reshape(-1, self.d_model).t() @ d_proj.reshape(-1, self.d_in_proj)).float()
        dx = torch.matmul(d_proj, w_in.t())
        grads = dict(in_proj=g_in_proj, dt_bias=g_dt_bias, B_bias=g_B_bias, C_bias=g_C_bias, B_norm=g_B_norm,
                     C_norm=g_C_norm, D=g_D, out_norm=g_out_norm, out_proj=g_out_proj)
        return dx, [grads[k] for k in PARAM_NAMES]

    __call__ = forward


class _LayerTrain(torch.autograd.Function):
    """Mamba3Layer.train_forward: x and the layer's float32 parameters in, the layer's
    output out; the backward returns the gradient of x (in x's dtype) and of each
    parameter (float32)."""

    @staticmethod
    def forward(ctx, layer, x, *params):
        w_in = params[PARAM_NAMES.index("in_proj")].to(layer.dtype).contiguous()
        w_out = params[PARAM_NAMES.index("out_proj")].to(layer.dtype).contiguous()
        unbatched = x.dim() == 2
        out, saved, _ = layer._run(x, w_in, w_out, keep=True)
        ctx.layer, ctx.saved, ctx.w = layer, saved, (w_in, w_out)
        ctx.unbatched, ctx.x_dtype = unbatched, x.dtype
        return out

    @staticmethod
    def backward(ctx, dout):
        layer = ctx.layer
        dx, dparams = layer._backward(ctx.saved, dout, *ctx.w)
        ctx.saved = None
        dx = dx.to(ctx.x_dtype)
        return (None, dx[0] if ctx.unbatched else dx, *dparams)


def init_params(d_model: int, seed: int, device, d_state: int = 128, expand: int = 2, headdim: int = 64,
                rope_fraction: float = 0.5, dt_min: float = 0.001, dt_max: float = 0.1) -> Dict[str, torch.Tensor]:
    """Random float32 parameters with the reference's initialisers (mamba3.py:145-183),
    generated on the device."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    d_inner_target = expand * d_model
    hd = min(headdim, d_inner_target)
    nh = max(1, d_inner_target // hd)
    split = int(d_state * rope_fraction)
    split -= split % 2
    R = split // 2
    di = nh * hd
    dproj = 2 * di + 2 * d_state + 3 * nh + R
    f = dict(device=device, dtype=torch.float32)
    u = torch.rand(nh, generator=g, **f)
    dt = torch.exp(u * (math.log(dt_max) - math.log(dt_min)) + math.log(dt_min)).clamp_min(1e-4)
    return dict(in_proj=torch.randn(d_model, dproj, generator=g, **f) / math.sqrt(d_model),
                dt_bias=dt + torch.log(-torch.expm1(-dt)), B_bias=torch.ones(nh, d_state, **f),
                C_bias=torch.ones(nh, d_state, **f), B_norm=torch.ones(d_state, **f), C_norm=torch.ones(d_state, **f),
                D=torch.ones(nh, **f), out_norm=torch.ones(di, **f),
                out_proj=torch.randn(di, d_model, generator=g, **f) / math.sqrt(di))
