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
