"""Decode state update on the GPU vs the CPU oracle's rnn_step (float64).

Covers both input dtypes, the reference's mode knobs (mamba3.py:28-45),
multi-step accumulation, the headline decode shape (config 4: B=512, H=32,
P=64, N=128) over its whole 256-step chain (three batch rows checked), and the prefill -> decode handoff:
decoding T tokens after a prefill of L tokens equals a prefill of L + T
(chunked == recurrent, test_backbone_contracts.py:81-111).
"""
import numpy as np
import pytest

from _util import I, M, oracle_scan, rel, to_dev

pytestmark = pytest.mark.gpu


def _dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def _decode(B, H, N, P, R, steps, seed, bf16, angle_mode="wrapped", diag_mode="current",
            out_dtype=None):
    import torch
    from mamba3_rocm import rnn_step_hip
    d = I.decode_inputs(B, H, N, P, R, steps, seed=seed, bf16=bf16)
    io = torch.bfloat16 if bf16 else torch.float32
    carry = tuple(_dev(d[k]) for k in ("theta", "h", "k_prev", "v_prev"))
    ref_carry = tuple(d[k].astype(np.float64) for k in ("theta", "h", "k_prev", "v_prev"))
    out_dtype = out_dtype or torch.float32
    ys, refs = [], []
    for s in range(steps):
        t_in = (_dev(d["x"][s], io), _dev(d["z"][s], io), _dev(d["Bt"][s], io), _dev(d["Ct"][s], io),
                _dev(d["adt"][s]), _dev(d["dt"][s]), _dev(d["trap"][s]), _dev(d["ang"][s]))
        carry, y = rnn_step_hip(carry, t_in, _dev(d["B_bias"]), _dev(d["C_bias"]), _dev(d["D"]),
                                angle_mode=angle_mode, diag_mode=diag_mode, out_dtype=out_dtype)
        ys.append(y.float().cpu().numpy())
        ref_in = tuple(d[k][s] for k in ("x", "z", "Bt", "Ct", "adt", "dt", "trap", "ang"))
        ref_carry, yr = M.rnn_step(ref_carry, ref_in, d["B_bias"], d["C_bias"], d["D"],
                                   angle_mode=angle_mode, diag_mode=diag_mode)
        refs.append(yr)
    torch.cuda.synchronize()
    got_carry = tuple(c.cpu().numpy() for c in carry)
    return np.stack(ys), np.stack(refs), got_carry, ref_carry


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("B,H,N,P,R", [(4, 3, 128, 64, 32), (2, 2, 64, 32, 16), (3, 2, 16, 16, 4),
                                         (2, 2, 4, 4, 1), (2, 2, 256, 32, 64), (2, 1, 32, 128, 0)])
def test_decode_matches_oracle(B, H, N, P, R, bf16):
    y, yr, c, cr = _decode(B, H, N, P, R, steps=8, seed=11, bf16=bf16)
    err = rel(y, yr)
    print(f"decode {(B, H, N, P, R)} bf16={bf16} y rel={err:.3e}")
    assert err <= 1e-4
    for a, b in zip(c, cr):
        if b.size:
            assert rel(a, b) <= 1e-4


@pytest.mark.parametrize("angle_mode,diag_mode", [("legacy_unbounded", "current"),
                                                  ("wrapped", "legacy_double"),
                                                  ("legacy_unbounded", "legacy_double")])
def test_decode_modes(angle_mode, diag_mode):
    y, yr, c, cr = _decode(2, 2, 64, 64, 16, steps=6, seed=12, bf16=True,
                           angle_mode=angle_mode, diag_mode=diag_mode)
    assert rel(y, yr) <= 1e-4
    assert rel(c[0], cr[0]) <= 1e-4


def test_decode_legacy_double_bitwise_repeatable():
    """legacy_double's QK dot is summed in a fixed order (no atomics): repeated steps
    from the same carry give bitwise-identical outputs."""
    ys = [_decode(2, 3, 128, 64, 32, steps=3, seed=14, bf16=True, diag_mode="legacy_double")[0]
          for _ in range(3)]
    assert all(np.array_equal(ys[0], y) for y in ys[1:])


def test_decode_bf16_output():
    import torch
    y, yr, _, _ = _decode(2, 2, 128, 64, 32, steps=4, seed=13, bf16=True, out_dtype=torch.bfloat16)
    assert rel(y, yr) <= 1e-2


def test_decode_headline_shape_subset():
    """Config 4 shape (B=512, H=32, P=64, N=128), 3 steps, rows 0, 200, 511 checked."""
    import torch
    from mamba3_rocm import rnn_step_hip
    B, H, N, P, R, steps = 512, 32, 128, 64, 32, 3
    d = I.decode_inputs(B, H, N, P, R, steps, seed=4, bf16=True)
    carry = tuple(_dev(d[k]) for k in ("theta", "h", "k_prev", "v_prev"))
    rows = [0, 200, 511]
    ref_carry = tuple(d[k][rows].astype(np.float64) for k in ("theta", "h", "k_prev", "v_prev"))
    for s in range(steps):
        t_in = (_dev(d["x"][s], torch.bfloat16), _dev(d["z"][s], torch.bfloat16),
                _dev(d["Bt"][s], torch.bfloat16), _dev(d["Ct"][s], torch.bfloat16),
                _dev(d["adt"][s]), _dev(d["dt"][s]), _dev(d["trap"][s]), _dev(d["ang"][s]))
        carry, y = rnn_step_hip(carry, t_in, _dev(d["B_bias"]), _dev(d["C_bias"]), _dev(d["D"]))
        ref_in = tuple(d[k][s][rows] for k in ("x", "z", "Bt", "Ct", "adt", "dt", "trap", "ang"))
        ref_carry, yr = M.rnn_step(ref_carry, ref_in, d["B_bias"], d["C_bias"], d["D"])
        assert rel(y.cpu().numpy()[rows], yr) <= 1e-4
    assert rel(carry[1].cpu().numpy()[rows], ref_carry[1]) <= 1e-4


def test_decode_config4_full_chain():
    """Config 4 as BASELINE states it: B=512, H=32, P=64, N=128, R=32, 256 consecutive
    steps in place on one carry (bf16 step inputs, float32 state), generated on the
    device with the configuration's distributions.  Rows 0, 200 and 511 follow the
    float64 rnn_step (mamba3.py:498-562) over the whole chain: y at every step
    (steps 1, 128 and 256 named in the message) and the final carry, at the float32
    bar 1e-4."""
    import math
    import torch
    from mamba3_rocm import rnn_step_hip
    B, H, N, P, R, T = 512, 32, 128, 64, 32, 256
    rows = [0, 200, 511]
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    f = dict(device="cuda", dtype=torch.float32, generator=g)
    sN = 1.0 / math.sqrt(N)
    carry = (torch.rand(B, H, R, **f) * 2 * math.pi, torch.randn(B, H, P, N, **f) * 0.1,
             torch.randn(B, H, N, **f) * sN, torch.randn(B, H, P, **f))
    bf = torch.bfloat16
    A = -torch.exp(torch.rand(H, **f) * math.log(16.0))
    Bb, Cb, D = torch.randn(H, N, **f) * sN, torch.randn(H, N, **f) * sN, torch.randn(H, **f)
    host = lambda t: t.double().cpu().numpy()  # noqa: E731
    ref_carry = tuple(host(c[rows]) for c in carry)
    ptrs = [c.data_ptr() for c in carry]
    print(f"case decode config 4 full chain B={B} H={H} steps={T}", flush=True)
    worst = {}
    for s in range(T):
        x = torch.randn(B, H, P, **f).to(bf)
        z = torch.randn(B, H, P, **f).to(bf)
        bt = (torch.randn(B, H, N, **f) * sN).to(bf)
        ct = (torch.randn(B, H, N, **f) * sN).to(bf)
        dt = torch.nn.functional.softplus(torch.randn(B, H, **f) * 0.5 - 2.0)
        adt = A[None, :] * dt
        trap = torch.sigmoid(torch.rand(B, H, **f))
        ang = (torch.rand(B, H, R, **f) * 2 - 1) * math.pi
        carry, y = rnn_step_hip(carry, (x, z, bt, ct, adt, dt, trap, ang), Bb, Cb, D)
        ref_in = tuple(host(t[rows]) for t in (x, z, bt, ct, adt, dt, trap, ang))
        ref_carry, yr = M.rnn_step(ref_carry, ref_in, host(Bb), host(Cb), host(D))
        err = rel(y[rows].cpu().numpy(), yr)
        worst[s + 1] = err
        assert err <= 1e-4, f"y at step {s + 1}: rel {err:.2e}"
    assert [c.data_ptr() for c in carry] == ptrs, "the carry was not updated in place"
    names = ("theta", "h", "k_prev", "v_prev")
    cerr = {n: rel(c[rows].cpu().numpy(), r) for n, c, r in zip(names, carry, ref_carry)}
    # the angle state is wrapped into [0, 2 pi): compare it on the circle, so that a value
    # next to the wrap that rounding puts on the other side is not an error of 2 pi
    dth = carry[0][rows].double().cpu().numpy() - ref_carry[0]
    cerr["theta"] = float(np.abs((dth + np.pi) % (2 * np.pi) - np.pi).max() / (2 * np.pi))
    print(f"  y rel at steps 1/128/256: {worst[1]:.1e} {worst[128]:.1e} {worst[256]:.1e}; "
          f"max {max(worst.values()):.1e}; final carry " +
          " ".join(f"{k}:{v:.1e}" for k, v in cerr.items()), flush=True)
    bad = {k: v for k, v in cerr.items() if v > 1e-4}
    assert not bad, f"final carry above 1e-4: {bad}"


@pytest.mark.parametrize("bf16", [False, True])
def test_prefill_then_decode_equals_longer_prefill(bf16):
    """Prefill L tokens with the carry out, decode T more with rnn_step_hip:
    the decoded outputs equal the last T outputs of the oracle over L + T."""
    import torch
    from mamba3_rocm import mamba3_siso_hip_carry, rnn_step_hip
    B, Lt, T, H, N, P, R = 2, 200, 12, 2, 128, 64, 32
    L = Lt - T
    d = I.scan_inputs(B, Lt, H, N, P, R, seed=14, bf16=bf16)
    io = torch.bfloat16 if bf16 else torch.float32
    t = to_dev(d, io)
    pre = {k: (v[:, :L] if k in ("Q", "K", "V", "Z", "Angles") else
               v[:, :, :L] if k in ("ADT", "DT", "Trap") else v) for k, v in t.items()}
    y_pre, carry = mamba3_siso_hip_carry(pre["Q"], pre["K"], pre["V"], pre["ADT"], pre["DT"],
                                         pre["Trap"], pre["Q_bias"], pre["K_bias"], pre["Angles"],
                                         pre["D"], pre["Z"], 64)
    ys = []
    for s in range(L, Lt):
        t_in = (t["V"][:, s], t["Z"][:, s], t["K"][:, s], t["Q"][:, s], t["ADT"][:, :, s],
                t["DT"][:, :, s], torch.sigmoid(t["Trap"][:, :, s]), t["Angles"][:, s])
        carry, y = rnn_step_hip(carry, t_in, t["K_bias"], t["Q_bias"], t["D"])
        ys.append(y)
    torch.cuda.synchronize()
    ref = oracle_scan(d, 64)
    tol = 2e-2 if bf16 else 1e-4
    assert rel(y_pre.float().cpu().numpy(), ref[:, :L]) <= tol
    dec = torch.stack(ys, dim=1).float().cpu().numpy()
    err = rel(dec, ref[:, L:])
    print(f"prefill->decode bf16={bf16} rel={err:.3e}")
    assert err <= tol
