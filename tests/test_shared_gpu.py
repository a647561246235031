"""The fused path's contract (B, C and angle rates shared over heads) on the GPU.

The reference pins mamba3_ssd_chunked_pallas against the per-head scan called
with Q, K and angles repeated over heads, and its gradients against jax.grad of
that scan with the repeated inputs' gradients summed over heads
(test_mamba3_pallas_ssd.py:55-72, 86-128).  Same here: the oracle sees the
repeated inputs; forward bars as for the scan (fp32 1e-4, bf16 2e-2), gradient
bars as for the backward (fp32 2e-5, bf16 3e-2).
"""
import numpy as np
import pytest

from _util import I, oracle_scan, rel
from oracle import mamba3_vjp as V

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _inputs(B, L, H, N, P, R, seed, bf16):
    d = I.scan_inputs(B, L, H, N, P, R, seed=seed, Hqk=1, bf16=bf16)
    shared = dict(d)
    shared["Q"], shared["K"] = d["Q"][:, :, 0], d["K"][:, :, 0]          # (B, L, N)
    shared["Angles"] = np.ascontiguousarray(d["Angles"][:, :, 0])       # (B, L, R)
    rep = dict(d)
    rep["Angles"] = np.repeat(shared["Angles"][:, :, None], H, axis=2)  # what the oracle sees
    return shared, rep


def _dev(d, dtype):
    torch = _torch()
    out = {}
    for k, v in d.items():
        t = torch.from_numpy(np.ascontiguousarray(v)).to("cuda")
        out[k] = t.to(dtype) if k in ("Q", "K", "V", "Z") else t
    return out


def _call(t, chunk, seq_split=True):
    from mamba3_rocm import mamba3_ssd_chunked_shared_hip
    return mamba3_ssd_chunked_shared_hip(t["Q"], t["K"], t["V"], t["ADT"], t["DT"], t["Trap"], t["Angles"],
                                         t["Q_bias"], t["K_bias"], t["D"], t["Z"], chunk_size=chunk,
                                         seq_split=seq_split)


@pytest.mark.parametrize("B,L,H,N,P,R,CS,bf16", [
    (2, 300, 4, 128, 64, 32, 64, True),
    (1, 1061, 3, 128, 64, 32, 64, True),     # B*H small: the sequence split runs
    (1, 200, 4, 64, 32, 16, 32, False),
])
def test_shared_forward_matches_repeated_oracle(B, L, H, N, P, R, CS, bf16):
    torch = _torch()
    from mamba3_rocm import mamba3_siso_hip
    shared, rep = _inputs(B, L, H, N, P, R, seed=41, bf16=bf16)
    dt = torch.bfloat16 if bf16 else torch.float32
    t = _dev(shared, dt)
    y = _call(t, CS).float().cpu().numpy()
    ref = oracle_scan(rep, CS)
    err = rel(y, ref)
    print(f"shared fwd {(B, L, H, N, P, R, CS)} bf16={bf16} rel={err:.3e}", flush=True)
    assert err <= (2e-2 if bf16 else 1e-4)
    # the per-head kernel on the repeated angles computes the same numbers
    tr = _dev(rep, dt)
    y2 = mamba3_siso_hip(tr["Q"], tr["K"], tr["V"], tr["ADT"], tr["DT"], tr["Trap"], tr["Q_bias"],
                         tr["K_bias"], tr["Angles"], tr["D"], tr["Z"], CS).float().cpu().numpy()
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("B,L,H,N,P,R,bf16", [
    (1, 200, 4, 128, 64, 32, True),
    (2, 90, 2, 64, 32, 16, False),
])
def test_shared_gradients_match_oracle(B, L, H, N, P, R, bf16, bwd_route):
    torch = _torch()
    shared, rep = _inputs(B, L, H, N, P, R, seed=42, bf16=bf16)
    dt = torch.bfloat16 if bf16 else torch.float32
    t = _dev(shared, dt)
    names = ("Q", "K", "V", "ADT", "DT", "Trap", "Angles", "Q_bias", "K_bias", "D", "Z")
    leaves = {k: t[k].clone().requires_grad_(True) for k in names}
    cot = V.cotangent(B, L, H, P, seed=43)
    if bf16:
        cot = I.bf16_round(cot)
    y = _call(leaves, 64)
    y.backward(torch.from_numpy(cot).to("cuda").to(dt))
    _, ref = V.vjp(rep, cot, 16)
    ref = dict(zip(V.NAMES, ref))
    ref["Q"], ref["K"] = ref["Q"][:, :, 0], ref["K"][:, :, 0]          # Hqk = 1: summed over heads
    ref["Angles"] = ref["Angles"].sum(axis=2)                           # repeated rates: sum over heads
    tol = 3e-2 if bf16 else 2e-5
    errs = {k: rel(leaves[k].grad.float().cpu().numpy(), ref[k]) for k in names}
    print(f"shared bwd {(B, L, H, N, P, R)} bf16={bf16} " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()),
          flush=True)
    assert all(v <= tol for v in errs.values()), errs


def test_per_head_angles_take_the_per_head_path():
    """angles (L, nh, R) are accepted (the fused path's third form)."""
    torch = _torch()
    B, L, H, N, P, R = 1, 130, 2, 128, 64, 32
    shared, rep = _inputs(B, L, H, N, P, R, seed=44, bf16=True)
    t = _dev(shared, torch.bfloat16)
    t["Angles"] = torch.from_numpy(rep["Angles"]).to("cuda")
    y = _call(t, 64).float().cpu().numpy()
    assert rel(y, oracle_scan(rep, 64)) <= 2e-2


@pytest.mark.parametrize("B,L,H,N,P,R,bf16", [
    (2, 200, 4, 128, 64, 32, True),
    (1, 1100, 3, 128, 64, 32, True),      # B*H small: the training forward takes the sequence split
    (1, 150, 4, 128, 64, 32, False),
    (2, 90, 2, 64, 32, 16, False),
])
def test_shared_training_pair(B, L, H, N, P, R, bf16, bwd_route):
    """The fused path's training pair (the forward that saves the chunk states, the
    backward that reads them, as the reference's chunk_scan_fwd_rule /
    chunk_scan_bwd_rule, mamba3_pallas.py:602-645): the forward's output equals the
    plain forward bitwise, and the gradients equal the recomputing backward's
    (bitwise where both produce the chunk states with the same kernel code: bf16
    without the split, float32 at d_state 128 without Z on the walk) and the
    repeated-input oracle within the bars."""
    torch = _torch()
    from mamba3_rocm import mamba3_ssd_chunked_shared_hip_bwd, mamba3_ssd_chunked_shared_hip_fwd_train
    shared, rep = _inputs(B, L, H, N, P, R, seed=45, bf16=bf16)
    dt = torch.bfloat16 if bf16 else torch.float32
    t = _dev(shared, dt)
    names = ("Q", "K", "V", "ADT", "DT", "Trap", "Angles", "Q_bias", "K_bias", "D", "Z")
    args = tuple(t[k] for k in names)
    print(f"case shared training pair {(B, L, H, N, P, R)} bf16={bf16} route={bwd_route}", flush=True)
    out_tr, saved = mamba3_ssd_chunked_shared_hip_fwd_train(*args, chunk_size=64)
    out = _call(t, 64)
    torch.cuda.synchronize()
    assert saved is not None
    assert torch.equal(out_tr, out), "training forward output differs from the forward"
    cot = V.cotangent(B, L, H, P, seed=46)
    if bf16:
        cot = I.bf16_round(cot)
    dout = torch.from_numpy(cot).to("cuda").to(dt)
    g_saved = mamba3_ssd_chunked_shared_hip_bwd(*args, dout, chunk_size=64, saved=saved)
    g_re = mamba3_ssd_chunked_shared_hip_bwd(*args, dout, chunk_size=64)
    torch.cuda.synchronize()
    _, ref = V.vjp(rep, cot, 16)
    ref = dict(zip(V.NAMES, ref))
    ref["Q"], ref["K"] = ref["Q"][:, :, 0], ref["K"][:, :, 0]
    ref["Angles"] = ref["Angles"].sum(axis=2)
    split = L > 1000
    exact = (bf16 and not split) or (not bf16 and N == 128 and bwd_route == "chunks")
    tol = 3e-2 if bf16 else 2e-5
    for k, a, b in zip(names, g_saved, g_re):
        a, b = a.float().cpu().numpy(), b.float().cpu().numpy()
        if exact and k != "Z":
            assert np.array_equal(a, b), f"d{k}: saved-state backward differs from the recompute"
        else:
            assert rel(a, b) <= (1e-2 if bf16 else 1e-5), (k, rel(a, b))
        assert rel(a, ref[k]) <= tol, (k, rel(a, ref[k]))


@pytest.mark.parametrize("io_bf16", [False, True])
def test_shared_compute_dtype_knob(io_bf16, monkeypatch):
    """MAMBA3_PALLAS_DTYPE sets the operand dtype of the fused path's kernels
    (mamba3_pallas.py:112-122, 838-839): with float32 inputs and the knob at
    bfloat16 the result is the bf16 kernel's on the inputs rounded to bf16, returned
    in float32; with bf16 inputs and the knob at float32 it is the float32 kernel's on
    the widened inputs, returned in bf16.  Gradients under the knob follow the oracle
    at the compute dtype's bar."""
    torch = _torch()
    B, L, H, N, P, R = 2, 200, 4, 128, 64, 32
    shared, rep = _inputs(B, L, H, N, P, R, seed=47, bf16=True)
    io = torch.bfloat16 if io_bf16 else torch.float32
    cdt = torch.float32 if io_bf16 else torch.bfloat16
    t = _dev(shared, io)
    monkeypatch.delenv("MAMBA3_PALLAS_DTYPE", raising=False)
    y_plain = _call(_dev(shared, cdt), 64)
    monkeypatch.setenv("MAMBA3_PALLAS_DTYPE", "float32" if cdt == torch.float32 else "bfloat16")
    y = _call(t, 64)
    torch.cuda.synchronize()
    assert y.dtype == io
    assert torch.equal(y, y_plain.to(io)), "the knob's result differs from the kernel of its dtype"
    names = ("Q", "K", "V", "ADT", "DT", "Trap", "Angles", "Q_bias", "K_bias", "D", "Z")
    leaves = {k: t[k].clone().requires_grad_(True) for k in names}
    cot = I.bf16_round(V.cotangent(B, L, H, P, seed=48))
    _call(leaves, 64).backward(torch.from_numpy(cot).to("cuda").to(io))
    _, ref = V.vjp(rep, cot, 16)
    ref = dict(zip(V.NAMES, ref))
    ref["Q"], ref["K"] = ref["Q"][:, :, 0], ref["K"][:, :, 0]
    ref["Angles"] = ref["Angles"].sum(axis=2)
    errs = {k: rel(leaves[k].grad.float().cpu().numpy(), ref[k]) for k in names}
    print(f"shared knob io_bf16={io_bf16} " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    tol = 3e-2 if cdt == torch.bfloat16 else 1e-2    # bf16 inputs: the gradients are rounded to bf16
    assert all(v <= tol for v in errs.values()), errs
