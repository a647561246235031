"""The mixer layer's backward (Mamba3Layer.train_forward).

* float32 compute against central finite differences of the float64 layer oracle
  (oracle/mamba3_layer.py): for a fixed output cotangent g, f(theta) =
  sum(g * layer(theta)); for each input (x and every parameter) a random direction u
  of its shape, and the directional derivative <grad, u> from the backward against
  (f(theta + e u) - f(theta - e u)) / 2e.  A mistake in any one gradient fails its
  own direction.  Bar 1e-3: the float64 difference quotient is exact to about 1e-8,
  the float32 scan's gradients are within 2e-5 of the oracle's, and the layer's norms
  add a few multiples of that.
* bf16 compute against the float32 backward of the same layer (same parameters and
  input), every gradient within the reference's bf16 gradient bar of 1e-1
  (tests/integration/test_mamba3_pallas_gpu.py:66-69), relative in norm.  A
  difference quotient of the bf16 layer itself would measure its rounding steps.
* The layer's in-place training pair (m3_layer_scan_train, m3_layer_scan_bwd: x and z
  read from the projection rows, dV and dZ written into the gradient's rows) against
  the contiguous pair on copies, bitwise: only the addressing differs.
"""
import numpy as np
import pytest

from _util import rel
from oracle import mamba3_layer as ML

pytestmark = pytest.mark.gpu

NAMES = ("in_proj", "dt_bias", "B_bias", "C_bias", "B_norm", "C_norm", "D", "out_norm", "out_proj")


def _grads(p, x, g, d_model, N, headdim, dtype, path):
    """Output and gradients (x first, then NAMES) of train_forward, as float64 numpy.
    train_forward runs the scan's training pair on copies of x and z; its output must
    equal the plain forward's (route ``path``) bitwise."""
    import torch
    from mamba3_rocm import Mamba3Layer
    params = {k: torch.from_numpy(v).cuda().requires_grad_(True) for k, v in p.items()}
    layer = Mamba3Layer(params, d_model, d_state=N, headdim=headdim, dtype=dtype)
    for k in NAMES:
        assert layer.params[k] is params[k], "the layer keeps the caller's float32 parameters"
    xt = torch.from_numpy(x).cuda().requires_grad_(True)
    out = layer.train_forward(xt)
    assert layer.last_scan == "train_" + path
    (out.float() * torch.from_numpy(g).float().cuda()).sum().backward()
    torch.cuda.synchronize()
    # the differentiable forward is the layer's forward
    plain = layer(torch.from_numpy(x).cuda())
    assert layer.last_scan == path
    assert torch.equal(out, plain), "train_forward's output differs from the forward's"

    grads = {"x": xt.grad.float().cpu().numpy().astype(np.float64)}
    for k in NAMES:
        assert params[k].grad is not None and params[k].grad.dtype == torch.float32, k
        grads[k] = params[k].grad.cpu().numpy().astype(np.float64)
        assert np.isfinite(grads[k]).all(), k
    assert np.isfinite(grads["x"]).all()
    return grads


def _setup(B, L, d_model, N, headdim):
    p = ML.init_params(d_model, seed=61, d_state=N, headdim=headdim)
    rng = np.random.default_rng(62)
    x = rng.standard_normal((B, L, d_model)).astype(np.float32)
    g = rng.standard_normal((B, L, d_model))
    return p, x, g


@pytest.mark.parametrize("B,L,d_model,N,headdim,path", [
    (2, 150, 64, 64, 32, "in_place"),      # the chunked float32 kernels at d_state 64
    (2, 200, 128, 128, 64, "in_place"),    # the model's geometry per head (812-wide float32 rows)
])
def test_layer_backward_f32_matches_finite_differences(B, L, d_model, N, headdim, path):
    import torch
    p, x, g = _setup(B, L, d_model, N, headdim)
    grads = _grads(p, x, g, d_model, N, headdim, torch.float32, path)
    errs = {}
    for i, name in enumerate(("x",) + NAMES):
        base = x if name == "x" else p[name]
        u = np.random.default_rng(100 + i).standard_normal(base.shape)
        e = 1e-3 * max(1.0, float(np.abs(base).max()))

        def at(s):
            pp = dict(p)
            xx = x
            if name == "x":
                xx = x + s * e * u
            else:
                pp[name] = p[name] + s * e * u
            return float(np.sum(g * ML.layer_forward(pp, xx, d_state=N, headdim=headdim)))
        fd = (at(1.0) - at(-1.0)) / (2.0 * e)
        an = float(np.sum(grads[name] * u))
        errs[name] = abs(an - fd) / max(abs(fd), 1e-12)
    print(f"layer bwd f32 {(B, L, d_model, N, headdim)}: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()),
          flush=True)
    bad = {k: v for k, v in errs.items() if v > 1e-3}
    assert not bad, f"directional derivatives above 1e-3: {bad}"


@pytest.mark.parametrize("B,L,d_model,N,headdim,path", [
    (2, 330, 256, 128, 64, "in_place"),    # 1336-wide bf16 rows: x and z read in place
    (2, 200, 128, 128, 64, "copies"),      # 812-wide bf16 rows: x and z copied
    (1, 1100, 256, 128, 64, "in_place"),   # 8 pairs: the scan's sequence splits, forward and backward
])
def test_layer_backward_bf16_matches_f32(B, L, d_model, N, headdim, path):
    import torch
    p, x, g = _setup(B, L, d_model, N, headdim)
    ref = _grads(p, x, g, d_model, N, headdim, torch.float32, "in_place")
    got = _grads(p, x, g, d_model, N, headdim, torch.bfloat16, path)
    errs = {k: rel(got[k], ref[k]) for k in ref}
    print(f"layer bwd bf16 vs f32 {(B, L, d_model, N, headdim)}: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()),
          flush=True)
    bad = {k: v for k, v in errs.items() if v > 1e-1}
    assert not bad, f"bf16 gradients above 1e-1 of the float32 ones: {bad}"


def _ptr(t):
    return None if t is None else t.data_ptr()


@pytest.mark.parametrize("B,L,H,bf16", [
    (2, 330, 8, True),      # 16 pairs, short: the chunk-parallel route
    (1, 2100, 8, True),     # 8 pairs, long: the split walk and its adjoint pass
    (4, 256, 64, True),     # 256 pairs: the one-segment walk
    (2, 200, 4, False),     # float32 I/O, the chunk-parallel route
    (1, 2100, 8, False),    # float32, the split walk (dZ from the saved output before the gate)
    (4, 256, 64, False),    # float32, the one-segment walk
])
def test_layer_scan_pair_in_place_matches_contiguous(B, L, H, bf16):
    import torch
    from _util import I
    from mamba3_rocm import _lib, mamba3_ssd_chunked_shared_hip_bwd, mamba3_ssd_chunked_shared_hip_fwd_train
    N, P, R, CS = 128, 64, 32, 64
    dt = torch.bfloat16 if bf16 else torch.float32
    io = _lib.DTYPE_BF16 if bf16 else _lib.DTYPE_F32
    d = I.scan_inputs(B, L, H, N, P, R, seed=71, Hqk=1, bf16=bf16)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda")  # noqa: E731
    Q, K = dev(d["Q"][:, :, 0]).to(dt), dev(d["K"][:, :, 0]).to(dt)
    V, Z = dev(d["V"]).to(dt), dev(d["Z"]).to(dt)
    ADT, DT, Trap, Qb, Kb, D = (dev(d[k]) for k in ("ADT", "DT", "Trap", "Q_bias", "K_bias", "D"))
    Ang = dev(d["Angles"][:, :, 0])
    width = 2 * H * P + 2 * N + 3 * H + R
    rng = np.random.default_rng(72)
    proj = dev(rng.standard_normal((B, L, width)).astype(np.float32)).to(dt)
    proj[..., :H * P] = Z.reshape(B, L, H * P)
    proj[..., H * P:2 * H * P] = V.reshape(B, L, H * P)
    dout = dev(rng.standard_normal((B, L, H, P)).astype(np.float32)).to(dt)
    print(f"case layer scan pair in place {(B, L, H)} bf16={bf16}", flush=True)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    args = (Q, K, V, ADT, DT, Trap, Ang, Qb, Kb, D, Z)

    # forward with residuals
    out_c, saved_c = mamba3_ssd_chunked_shared_hip_fwd_train(*args, chunk_size=CS)
    assert saved_c is not None
    out_i = torch.empty_like(out_c)
    saved_i = torch.empty_like(saved_c)
    wsb = lib.m3_chunk_scan_ws_bytes(B, L, H, N, P, R, CS, io)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    _lib.check(lib.m3_layer_scan_train(_ptr(Q), _ptr(K), _ptr(proj), width, _ptr(ADT), _ptr(DT), _ptr(Trap),
                                       _ptr(Ang), _ptr(Qb), _ptr(Kb), _ptr(D), _ptr(out_i), B, L, H, N, P, R, CS, io,
                                       _ptr(saved_i), saved_i.numel(), ws.data_ptr() if wsb else None, wsb, st),
               "m3_layer_scan_train")
    torch.cuda.synchronize()
    assert torch.equal(out_i, out_c), "in-place training forward output"
    assert torch.equal(saved_i, saved_c), "in-place training forward residuals"

    names = ("Q", "K", "V", "ADT", "DT", "Trap", "Angles", "Q_bias", "K_bias", "D", "Z")
    f32 = dict(device="cuda", dtype=torch.float32)
    for with_saved in (True, False):
        ref = dict(zip(names, mamba3_ssd_chunked_shared_hip_bwd(*args, dout, chunk_size=CS,
                                                                saved=saved_c if with_saved else None)))
        g = dict(Q=torch.empty_like(Q), K=torch.empty_like(K), ADT=torch.empty(B, H, L, **f32),
                 DT=torch.empty(B, H, L, **f32), Trap=torch.empty(B, H, L, **f32), Angles=torch.empty(B, L, R, **f32),
                 Q_bias=torch.empty(H, N, **f32), K_bias=torch.empty(H, N, **f32), D=torch.empty(H, **f32))
        d_proj = torch.full_like(proj, 7.0)
        if with_saved:
            wsb = lib.m3_chunk_scan_bwd_saved_shared_ws_bytes(B, L, H, N, P, R, CS, io)
        else:
            wsb = lib.m3_chunk_scan_bwd_shared_ws_bytes(B, L, H, N, P, R, CS, io)
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        _lib.check(lib.m3_layer_scan_bwd(
            _ptr(Q), _ptr(K), _ptr(proj), width, _ptr(ADT), _ptr(DT), _ptr(Trap), _ptr(Ang), _ptr(Qb), _ptr(Kb),
            _ptr(D), _ptr(dout), _ptr(g["Q"]), _ptr(g["K"]), _ptr(d_proj), _ptr(g["ADT"]), _ptr(g["DT"]),
            _ptr(g["Trap"]), _ptr(g["Q_bias"]), _ptr(g["K_bias"]), _ptr(g["Angles"]), _ptr(g["D"]),
            B, L, H, N, P, R, CS, io, _ptr(saved_c) if with_saved else None, saved_c.numel() if with_saved else 0,
            ws.data_ptr(), wsb, st), "m3_layer_scan_bwd")
        torch.cuda.synchronize()
        g["Z"] = d_proj[..., :H * P].reshape(B, L, H, P)
        g["V"] = d_proj[..., H * P:2 * H * P].reshape(B, L, H, P)
        for k in names:
            assert torch.equal(g[k], ref[k].reshape(g[k].shape)), f"d{k} (saved={with_saved})"
        assert bool((d_proj[..., 2 * H * P:] == 7.0).all()), "columns past x written"
