"""m3_layer_decode_step: the layer's decode step in one launch, against the two
launches it replaces, m3_layer_pre on the token (mamba3.py:203-268) followed by
m3_decode_step through rnn_step_hip (mamba3.py:498-562) with B, C and the angle rates
repeated over the heads and trap through torch's sigmoid.  Both paths run the same
arithmetic except the sigmoid (expf here, torch's kernel there), so the carries agree
to 1e-6 relative and y to 1e-6 in float32; bf16 y may differ by the rounding of an
element whose float32 value moved by an ulp (bar 4e-3, one bf16 ulp).  The decode
kernel itself is pinned against the float64 rnn_step oracle in test_decode_gpu.py, and
the layer's decode against the layer's forward in test_generate_gpu.py.
"""
import numpy as np
import pytest

from _util import rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bf16,angle_mode,diag_mode,N,P,R", [
    (True, "wrapped", "current", 128, 64, 32),
    (False, "wrapped", "current", 64, 32, 16),
    (True, "legacy_unbounded", "legacy_double", 128, 64, 32),
    (False, "legacy_unbounded", "current", 128, 64, 64),
    (False, "wrapped", "legacy_double", 64, 32, 0),
])
def test_layer_decode_step_matches_pre_then_decode(bf16, angle_mode, diag_mode, N, P, R):
    import torch
    from mamba3_rocm import _lib, rnn_step_hip
    B, H = 6, 5
    dt = torch.bfloat16 if bf16 else torch.float32
    io = _lib.DTYPE_BF16 if bf16 else _lib.DTYPE_F32
    d_in = 2 * H * P + 2 * N + 3 * H + R
    g = torch.Generator(device="cuda")
    g.manual_seed(101 + N + R)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=g)   # noqa: E731
    proj = rn(B, 1, d_in).to(dt)
    dt_bias, Bn_, Cn_ = rn(H) * 0.5, 1.0 + 0.1 * rn(N), 1.0 + 0.1 * rn(N)
    Bb, Cb, D = rn(H, N) * 0.3, rn(H, N) * 0.3, rn(H)
    carry0 = (rn(B, H, R) * 3.0, rn(B, H, P, N), rn(B, H, N), rn(B, H, P))
    A_floor, eps = 1e-4, 1e-6
    st = torch.cuda.current_stream().cuda_stream
    lib = _lib.load()
    print(f"case layer decode bf16={bf16} {angle_mode} {diag_mode} N={N} P={P} R={R}", flush=True)
    # the two launches
    c1 = tuple(t.clone() for t in carry0)
    Q, K = (torch.empty(B, 1, N, device="cuda", dtype=dt) for _ in range(2))
    V, Z = (torch.empty(B, 1, H, P, device="cuda", dtype=dt) for _ in range(2))
    ADT, DT, Trap = (torch.empty(B, H, 1, device="cuda") for _ in range(3))
    Ang = torch.empty(B, 1, max(R, 1), device="cuda")
    p = lambda t: t.data_ptr()   # noqa: E731
    _lib.check(lib.m3_layer_pre(p(proj), p(dt_bias), p(Bn_), p(Cn_), p(Q), p(K), p(V), p(Z), p(ADT), p(DT), p(Trap),
                                p(Ang), B, 1, H, P, N, R, A_floor, eps, io, st), "m3_layer_pre")
    inputs = (V[:, 0], Z[:, 0], K.expand(B, H, N), Q.expand(B, H, N), ADT[..., 0], DT[..., 0],
              torch.sigmoid(Trap[..., 0]), Ang[:, :, :R].expand(B, H, R))
    _, y1 = rnn_step_hip(c1, inputs, Bb, Cb, D, angle_mode=angle_mode, diag_mode=diag_mode, out_dtype=dt)
    # the one launch
    c2 = tuple(t.clone() for t in carry0)
    y2 = torch.empty(B, H, P, device="cuda", dtype=dt)
    _lib.check(lib.m3_layer_decode_step(p(proj), p(dt_bias), p(Bn_), p(Cn_), p(Bb), p(Cb), p(D), p(c2[0]), p(c2[1]),
                                        p(c2[2]), p(c2[3]), p(y2), B, H, P, N, R, A_floor, eps, io,
                                        1 if angle_mode == "wrapped" else 0, 1 if diag_mode == "legacy_double" else 0,
                                        st), "m3_layer_decode_step")
    torch.cuda.synchronize()
    errs = {n: rel(b.cpu().numpy(), a.cpu().numpy()) for n, a, b in zip(("theta", "ssm", "k", "v"), c1, c2)
            if a.numel()}
    ey = rel(y2.float().cpu().numpy(), y1.float().cpu().numpy())
    print("layer decode: y %.2e, " % ey + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v <= 1e-6 for v in errs.values()), errs
    assert ey <= (4e-3 if bf16 else 1e-6)
    assert np.isfinite(y2.float().cpu().numpy()).all()
