"""Backward of the prefill scan on the GPU vs the gradient oracle (parity gate).

Every one of the eleven input gradients is compared with torch autograd of the
float64 restatement (oracle/mamba3_vjp.py, the counterpart of the reference's
jax.grad pin, test_mamba3_pallas_ssd.py:108-128) on the same inputs and output
cotangent.  Metric: the reference's _rel (max abs error / max abs reference).
Bars: 2e-5 for float32 I/O (the reference's gradient bar); 3e-2 for bf16 I/O
(bf16 MFMA operands, float32 accumulation; the reference's bf16-I/O class).
"""
import numpy as np
import pytest

from _util import I, rel, to_dev
from oracle import mamba3_vjp as V

pytestmark = pytest.mark.gpu

F32_TOL = 2e-5
BF16_TOL = 3e-2


def _torch():
    import torch
    return torch


def _grads(d, cot, torch_dtype, no_d=False, no_z=False, chunk=64):
    torch = _torch()
    from mamba3_rocm import mamba3_siso_hip_bwd
    t = to_dev(d, torch_dtype)
    dout = torch.from_numpy(np.ascontiguousarray(cot)).to("cuda").to(torch_dtype)
    g = mamba3_siso_hip_bwd(t["Q"], t["K"], t["V"], t["ADT"], t["DT"], t["Trap"], t["Q_bias"],
                            t["K_bias"], t["Angles"], None if no_d else t["D"],
                            None if no_z else t["Z"], dout, chunk_size=chunk)
    torch.cuda.synchronize()
    return [None if x is None else x.float().cpu().numpy() for x in g]


def _check(B, L, H, Hqk, N, P, R, bf16, seed, no_d=False, no_z=False, chunk=64):
    torch = _torch()
    d = I.scan_inputs(B, L, H, N, P, R, seed=seed, Hqk=Hqk, bf16=bf16)
    cot = V.cotangent(B, L, H, P, seed=seed + 100)
    if bf16:
        cot = I.bf16_round(cot)
    print(f"case bwd {(B, L, H, Hqk, N, P, R)} bf16={bf16} no_d={no_d} no_z={no_z}", flush=True)
    got = _grads(d, cot, torch.bfloat16 if bf16 else torch.float32, no_d, no_z, chunk)
    _, ref = V.vjp(d, cot, 16, no_d=no_d, no_z=no_z)
    tol = BF16_TOL if bf16 else F32_TOL
    errs = {}
    for name, a, b in zip(V.NAMES, got, ref):
        if b is None:
            assert a is None, name
            continue
        assert a.shape == b.shape, (name, a.shape, b.shape)
        if b.size == 0:
            continue
        assert np.isfinite(a).all(), f"d{name} has non-finite entries"
        errs[name] = rel(a, b)
    print("  " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if v > tol}
    assert not bad, f"gradients above {tol}: {bad}"


BF16_SHAPES = [
    (1, 200, 2, 2, 128, 64, 32),     # model geometry, ragged L (several chunks)
    (2, 130, 4, 2, 128, 64, 32),     # GQA
    (1, 150, 2, 2, 128, 64, 64),     # rope on every state pair
    (1, 100, 2, 2, 128, 64, 0),      # no rope
    (1, 160, 2, 2, 64, 32, 16),
]


@pytest.mark.parametrize("B,L,H,Hqk,N,P,R", BF16_SHAPES)
def test_bf16_gradients_match_oracle(B, L, H, Hqk, N, P, R, bwd_route):
    _check(B, L, H, Hqk, N, P, R, bf16=True, seed=31)


F32_SHAPES = [
    (1, 150, 2, 2, 128, 64, 32),     # model geometry (Mamba3SSM hands its scan float32), ragged L
    (2, 100, 4, 2, 128, 64, 64),     # GQA, rope on every state pair
    (1, 150, 2, 2, 64, 32, 16),
    (2, 70, 4, 1, 64, 64, 16),       # GQA, L below two chunks
]


@pytest.mark.parametrize("B,L,H,Hqk,N,P,R", F32_SHAPES)
def test_f32_gradients_match_oracle(B, L, H, Hqk, N, P, R, bwd_route):
    _check(B, L, H, Hqk, N, P, R, bf16=False, seed=32)


def test_gradients_without_d_and_z(bwd_route):
    _check(1, 120, 2, 2, 128, 64, 32, bf16=True, seed=33, no_d=True, no_z=True)
    _check(1, 90, 2, 2, 64, 32, 16, bf16=False, seed=34, no_d=True, no_z=True)


def test_autograd_matches_functional_backward_and_is_deterministic(bwd_route):
    """mamba3_siso_hip under torch autograd (the custom_vjp, which runs the training
    pair) gives the functional training pair's gradients, bitwise, and the functional
    backward is bitwise repeatable; the recomputing backward agrees within rounding
    (the reverse walk's training-pair variant forms dZ from the saved output before
    the gate and is compiled apart, so its float contractions may differ)."""
    torch = _torch()
    from mamba3_rocm import mamba3_siso_hip, mamba3_siso_hip_bwd, mamba3_siso_hip_fwd_train
    B, L, H, N, P, R = 1, 140, 2, 128, 64, 32
    d = I.scan_inputs(B, L, H, N, P, R, seed=35, bf16=True)
    t = to_dev(d, torch.bfloat16)
    cot = torch.from_numpy(I.bf16_round(V.cotangent(B, L, H, P, seed=36))).to("cuda").to(torch.bfloat16)
    names = V.NAMES
    leaves = {k: t[k].clone().requires_grad_(True) for k in names}
    y = mamba3_siso_hip(*(leaves[k] for k in names), chunk_size=64)
    y.backward(cot)
    _, saved = mamba3_siso_hip_fwd_train(*(t[k] for k in names), chunk_size=64)
    g1 = mamba3_siso_hip_bwd(*(t[k] for k in names), cot, chunk_size=64, saved=saved)
    g2 = mamba3_siso_hip_bwd(*(t[k] for k in names), cot, chunk_size=64, saved=saved)
    g3 = mamba3_siso_hip_bwd(*(t[k] for k in names), cot, chunk_size=64)
    torch.cuda.synchronize()
    for k, a, b, c in zip(names, g1, g2, g3):
        assert torch.equal(a, b), f"d{k} differs between two calls"
        assert torch.equal(leaves[k].grad.to(a.dtype), a), f"autograd d{k} differs"
        ca, cc = a.float().cpu().numpy(), c.float().cpu().numpy()
        assert rel(ca, cc) <= 1e-2, (f"d{k}: training pair vs recompute", rel(ca, cc))


@pytest.mark.parametrize("B,L,H,Hqk,N,P,R,bf16", [
    (1, 1280, 16, 16, 128, 64, 32, True),   # 20 chunks x 16 heads = 320 items
    (1, 2600, 4, 4, 64, 32, 16, False),     # 82 chunks (of 32) x 4 heads = 328 items
])
def test_gradients_with_more_items_than_compute_units(B, L, H, Hqk, N, P, R, bf16, bwd_route):
    """More (chunk, b, h) items than compute units (longer sequences and more heads
    than the cases above): several waves of chunk-gradient workgroups per launch."""
    _check(B, L, H, Hqk, N, P, R, bf16=bf16, seed=37)


def _training_pair(B, L, H, Hqk, N, P, R, bf16, split, route, no_z=False, seed=41):
    """The training forward (the reference's mamba3_siso_fwd, which returns the
    per-chunk states with its output, mamba3_ops.py:788-818) gives the plain forward's
    output bitwise, and the backward that reads its saved chunk states gives the
    recomputing backward's gradients: bitwise where both produce the states with the
    same kernel code (bf16 one pass; float32 at d_state 128, whose state pass is the
    float32 kernel's), within rounding where the forward's states come from another
    kernel (float32 at d_state 64, the split), and within the bars against the
    oracle.  With Z on the reverse walk's route the comparison is within rounding:
    the walk's float32 training-pair variant forms dZ from the saved output before
    the gate (the reference's Out_v residual) where the recompute forms it from its
    own float32 product, and every training-pair variant is compiled apart."""
    torch = _torch()
    from mamba3_rocm import mamba3_siso_hip, mamba3_siso_hip_bwd, mamba3_siso_hip_fwd_train
    from mamba3_rocm import _lib
    d = I.scan_inputs(B, L, H, N, P, R, seed=seed, Hqk=Hqk, bf16=bf16)
    cot = V.cotangent(B, L, H, P, seed=seed + 1)
    tdt = torch.bfloat16 if bf16 else torch.float32
    if bf16:
        cot = I.bf16_round(cot)
    print(f"case training pair {(B, L, H, Hqk, N, P, R)} bf16={bf16} split={split} no_z={no_z} "
          f"route={route}", flush=True)
    t = to_dev(d, tdt)
    if no_z:
        t["Z"] = None
    args = tuple(t[k] for k in V.NAMES)
    io = _lib.DTYPE_BF16 if bf16 else _lib.DTYPE_F32
    assert (_lib.load().m3_chunk_scan_ws_bytes(B, L, H, N, P, R, 64, io) > 0) == split
    out_tr, saved = mamba3_siso_hip_fwd_train(*args, chunk_size=64)
    out = mamba3_siso_hip(*args, chunk_size=64)
    torch.cuda.synchronize()
    assert saved is not None, "the shape has a backward but no residual-writing forward"
    assert torch.equal(out_tr, out), "training forward output differs from the forward"
    dout = torch.from_numpy(np.ascontiguousarray(cot)).to("cuda").to(tdt)
    g_saved = mamba3_siso_hip_bwd(*args, dout, chunk_size=64, saved=saved)
    g_re = mamba3_siso_hip_bwd(*args, dout, chunk_size=64)
    torch.cuda.synchronize()
    _, ref = V.vjp(d, cot, 16, no_z=no_z)
    same_states = not split and (bf16 or N == 128)
    exact = same_states and (route == "chunks" or no_z or bf16)
    for name, a, b, r in zip(V.NAMES, g_saved, g_re, ref):
        if r is None:
            assert a is None and b is None, name
            continue
        a, b = a.float().cpu().numpy(), b.float().cpu().numpy()
        assert a.shape == r.shape, (name, a.shape, r.shape)
        if r.size == 0:          # dAngles without rope
            continue
        assert np.isfinite(a).all(), f"d{name} has non-finite entries"
        if exact and name != "Z":
            assert np.array_equal(a, b), f"d{name}: saved-state backward differs from the recompute"
        else:
            assert rel(a, b) <= (1e-2 if bf16 else 1e-5), (name, rel(a, b))
        assert rel(a, r) <= (BF16_TOL if bf16 else F32_TOL), (name, rel(a, r))


# Every shape whose forward writes the backward's residuals: the bf16 list of
# m3_scan_chunked.hip (M3_SAVE_SHAPES) and the float32 list of m3_scan_chunked_f32.hip
# (M3_F32_SAVE_SHAPES), as (N, P, R).
BF16_SAVE = [(128, 64, 32), (128, 64, 64), (128, 64, 0), (64, 64, 16), (64, 32, 16)]
F32_SAVE = [(128, 64, 32), (128, 64, 64), (64, 64, 16), (64, 32, 16)]
SAVE_CASES = [(N, P, R, True) for N, P, R in BF16_SAVE] + [(N, P, R, False) for N, P, R in F32_SAVE]


@pytest.mark.parametrize("no_z", [False, True], ids=["z", "no_z"])
@pytest.mark.parametrize("N,P,R,bf16", SAVE_CASES)
def test_training_pair_every_saved_shape(N, P, R, bf16, no_z, bwd_route):
    """Every residual-writing forward instantiation and both backward variants that
    read it (with Z the float32 walk's saved-output variant), ragged L over three
    chunks."""
    _training_pair(1, 150, 2, 2, N, P, R, bf16, False, bwd_route, no_z=no_z)


@pytest.mark.parametrize("B,L,H,Hqk,N,P,R,bf16,split", [
    (2, 130, 4, 2, 128, 64, 32, True, False),     # GQA
    (1, 1100, 3, 3, 128, 64, 32, True, True),     # the forward takes the sequence split
    (2, 100, 4, 2, 128, 64, 64, False, False),    # float32 GQA, rope on every pair
    (2, 90, 4, 1, 64, 64, 16, False, False),      # float32 GQA at d_state 64
    (1, 1100, 3, 3, 128, 64, 32, False, True),    # float32, the forward takes the sequence split
])
def test_training_pair_saved_states(B, L, H, Hqk, N, P, R, bf16, split, bwd_route):
    """The training pair with GQA and with a forward that takes the sequence split."""
    _training_pair(B, L, H, Hqk, N, P, R, bf16, split, bwd_route)
