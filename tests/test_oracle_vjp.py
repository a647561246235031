"""Pins of the gradient oracle (oracle/mamba3_vjp.py), CPU only.

The reference pins its backward against jax.grad of the XLA scan
(test_mamba3_pallas_ssd.py:108-128).  Here the torch float64 restatement is
pinned by: its forward equal to the numpy oracle; every gradient entry equal to
a central finite difference of the numpy oracle's loss (so a dropped term, a
wrong sign or a transposed operand in the restatement fails); gradients
independent of the chunk size (the chunked form is exact); every gradient
non-trivial on the test problem (test_mamba3_pallas_ssd.py:131-141).
"""
import numpy as np
import pytest

from oracle import inputs as I
from oracle import mamba3_ref as M
from oracle import mamba3_vjp as V


def _loss_np(d, cot, cs, no_d=False, no_z=False):
    y = M.mamba3_ssd_chunked_batched(
        d["Q"], d["K"], d["V"], d["ADT"], d["DT"], d["Trap"], d["Angles"], d["Q_bias"],
        d["K_bias"], None if no_d else d["D"], None if no_z else d["Z"], chunk_size=cs)
    return float(np.sum(y * cot))


def _small(seed, Hqk=1, L=11, H=2, N=8, P=4, R=2):
    d = I.scan_inputs(1, L, H, N, P, R, seed=seed, Hqk=Hqk)
    d = {k: np.asarray(v, dtype=np.float64) for k, v in d.items()}
    # larger angle rates and decay than the benchmark draws, so that every term matters
    d["Angles"] = d["Angles"] * 0.7
    return d


def test_forward_matches_numpy_oracle():
    for (B, L, H, Hqk, N, P, R, cs) in [(2, 70, 2, 2, 16, 8, 4, 16), (1, 45, 4, 2, 32, 16, 8, 8)]:
        d = I.scan_inputs(B, L, H, N, P, R, seed=7, Hqk=Hqk)
        cot = V.cotangent(B, L, H, P, seed=8)
        y, _ = V.vjp(d, cot, cs)
        ref = M.mamba3_ssd_chunked_batched(
            d["Q"], d["K"], d["V"], d["ADT"], d["DT"], d["Trap"], d["Angles"], d["Q_bias"],
            d["K_bias"], d["D"], d["Z"], chunk_size=cs)
        assert np.abs(y - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("no_d,no_z", [(False, False), (True, True)])
def test_gradients_match_finite_differences(no_d, no_z):
    d = _small(seed=3)
    B, L, H, P = 1, 11, 2, 4
    cs = 4
    cot = V.cotangent(B, L, H, P, seed=4).astype(np.float64)
    _, grads = V.vjp(d, cot, cs, no_d=no_d, no_z=no_z)
    eps = 1e-6
    for name, g in zip(V.NAMES, grads):
        if (name == "D" and no_d) or (name == "Z" and no_z):
            assert g is None
            continue
        fd = np.zeros_like(d[name])
        flat, gflat = d[name].reshape(-1), fd.reshape(-1)
        for i in range(flat.size):
            x0 = flat[i]
            flat[i] = x0 + eps
            up = _loss_np(d, cot, cs, no_d, no_z)
            flat[i] = x0 - eps
            dn = _loss_np(d, cot, cs, no_d, no_z)
            flat[i] = x0
            gflat[i] = (up - dn) / (2 * eps)
        err = np.abs(g - fd).max() / max(np.abs(fd).max(), 1e-12)
        assert err < 1e-6, f"d{name}: autograd vs finite differences {err:.2e}"


def test_gradients_independent_of_chunk_size():
    d = I.scan_inputs(1, 37, 2, 16, 8, 4, seed=5, Hqk=1)
    cot = V.cotangent(1, 37, 2, 8, seed=6)
    _, g4 = V.vjp(d, cot, 4)
    _, g16 = V.vjp(d, cot, 16)
    for name, a, b in zip(V.NAMES, g4, g16):
        assert np.abs(a - b).max() <= 1e-10 * max(1.0, np.abs(b).max()), name


def test_every_gradient_is_exercised():
    d = I.scan_inputs(1, 40, 2, 16, 8, 4, seed=11)
    cot = V.cotangent(1, 40, 2, 8, seed=12)
    _, grads = V.vjp(d, cot, 8)
    for name, g in zip(V.NAMES, grads):
        assert np.abs(g).max() > 1e-3, f"d{name} is (nearly) zero in the test problem"


def test_shift_invariances_of_angles_and_decay():
    """The backward's finishing pass relies on two exact facts of the operator: it
    depends on the rope angles and on the decay prefix A only through differences
    (theta_t - theta_s, A_t - A_s), so shifting every token's angle of one pair (by
    changing token 0's rate) or every A_t (token 0's adt) leaves the output unchanged,
    and the per-token d(theta) and dA sum to zero: dADT and dAngles vanish at token 0.
    A planted mistake that breaks the difference form (keys left unrotated) makes the
    forward check fail."""
    B, L, H, N, P, R = 1, 50, 2, 16, 8, 4
    d = I.scan_inputs(B, L, H, N, P, R, seed=21, Hqk=1)
    d = {k: np.asarray(v, dtype=np.float64) for k, v in d.items()}

    def fwd(dd):
        return M.mamba3_ssd_chunked_batched(
            dd["Q"], dd["K"], dd["V"], dd["ADT"], dd["DT"], dd["Trap"], dd["Angles"], dd["Q_bias"],
            dd["K_bias"], dd["D"], dd["Z"], chunk_size=8)

    y0 = fwd(d)
    e = dict(d)
    e["Angles"] = d["Angles"].copy()
    e["Angles"][:, 0, :, 1] += 0.9          # pair 1 of every head turns by a constant
    e["ADT"] = d["ADT"].copy()
    e["ADT"][:, :, 0] -= 0.7                # every A_t moves by the same amount
    assert np.abs(fwd(e) - y0).max() <= 1e-12 * np.abs(y0).max()
    # the same shift through a rope that is not a difference form changes the output
    rot, calls = M.apply_rope, [0]

    def q_only(x, c, s):                    # calls alternate Q, K: leave K unrotated
        calls[0] += 1
        return rot(x, c, s) if calls[0] % 2 else x
    try:
        M.apply_rope = q_only
        planted0, planted1 = fwd(d), fwd(e)
    finally:
        M.apply_rope = rot
    assert np.abs(planted1 - planted0).max() > 1e-3 * np.abs(y0).max()

    cot = V.cotangent(B, L, H, P, seed=22)
    _, g = V.vjp(d, cot, 8)
    gd = dict(zip(V.NAMES, g))
    assert np.abs(gd["ADT"][:, :, 0]).max() <= 1e-12 * np.abs(gd["ADT"]).max()
    assert np.abs(gd["Angles"][:, 0]).max() <= 1e-12 * np.abs(gd["Angles"]).max()
