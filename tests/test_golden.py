"""Golden fixtures (tests/golden/*.npz) against the oracle (CPU) and the HIP
kernels (GPU).  The fixtures are the oracle's float64 outputs on seeded
inputs, written by tests/golden/make_golden.py."""
import glob
import os

import numpy as np
import pytest

from _util import M, rel

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SCANS = sorted(glob.glob(os.path.join(GOLDEN, "scan_*.npz")))
DECODES = sorted(glob.glob(os.path.join(GOLDEN, "decode_*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_fixtures_present():
    assert len(SCANS) >= 3 and len(DECODES) >= 1


@pytest.mark.parametrize("path", SCANS, ids=os.path.basename)
def test_oracle_reproduces_scan_fixture(path):
    d = _load(path)
    B, L, H, N, P, R, CS, bf = (int(x) for x in d["dims"])
    y = M.mamba3_ssd_chunked_batched(d["Q"], d["K"], d["V"], d["ADT"], d["DT"], d["Trap"],
                                     d["Angles"], d["Q_bias"], d["K_bias"], d["D"], d["Z"],
                                     chunk_size=CS)
    assert rel(y, d["Y"]) < 1e-12


@pytest.mark.parametrize("path", DECODES, ids=os.path.basename)
def test_oracle_reproduces_decode_fixture(path):
    d = _load(path)
    carry = tuple(d[k].astype(np.float64) for k in ("theta", "h", "k_prev", "v_prev"))
    for s in range(int(d["dims"][5])):
        carry, y = M.rnn_step(carry, tuple(d[k][s] for k in ("x", "z", "Bt", "Ct", "adt", "dt",
                                                             "trap", "ang")),
                              d["B_bias"], d["C_bias"], d["D"])
        assert rel(y, d["Y"][s]) < 1e-12
    assert rel(carry[1], d["h_out"]) < 1e-12


@pytest.mark.gpu
@pytest.mark.parametrize("path", SCANS, ids=os.path.basename)
def test_hip_scan_matches_fixture(path):
    import torch
    from _util import hip_scan, to_dev
    d = _load(path)
    B, L, H, N, P, R, CS, bf = (int(x) for x in d["dims"])
    inputs = {k: d[k] for k in ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")}
    t = to_dev(inputs, torch.bfloat16 if bf else torch.float32)
    y = hip_scan(t, CS).float().cpu().numpy()
    err = rel(y, d["Y"])
    print(f"{os.path.basename(path)} rel={err:.3e}")
    assert err <= (2e-2 if bf else 1e-4)


@pytest.mark.gpu
@pytest.mark.parametrize("path", DECODES, ids=os.path.basename)
def test_hip_decode_matches_fixture(path):
    import torch
    from mamba3_rocm import rnn_step_hip
    d = _load(path)
    dev = lambda a, dt=None: (torch.from_numpy(np.ascontiguousarray(a)).cuda() if dt is None  # noqa: E731
                              else torch.from_numpy(np.ascontiguousarray(a)).cuda().to(dt))
    carry = tuple(dev(d[k]) for k in ("theta", "h", "k_prev", "v_prev"))
    bf = torch.bfloat16
    for s in range(int(d["dims"][5])):
        tin = (dev(d["x"][s], bf), dev(d["z"][s], bf), dev(d["Bt"][s], bf), dev(d["Ct"][s], bf),
               dev(d["adt"][s]), dev(d["dt"][s]), dev(d["trap"][s]), dev(d["ang"][s]))
        carry, y = rnn_step_hip(carry, tin, dev(d["B_bias"]), dev(d["C_bias"]), dev(d["D"]))
        assert rel(y.cpu().numpy(), d["Y"][s]) <= 1e-4
    assert rel(carry[1].cpu().numpy(), d["h_out"]) <= 1e-4
    assert rel(carry[2].cpu().numpy(), d["k_out"]) <= 1e-4
