"""Generate the golden fixtures in this directory from the CPU oracle.

The reference commits no golden vectors for the Mamba3 scan (its tests are
on-the-fly differential tests, tests/unit/test_mamba3_pallas_ssd.py:40-55),
and its JAX code cannot be imported here, so these vectors come from the
oracle in oracle/mamba3_ref.py (float64), itself pinned by tests/test_oracle.py.
Each file holds seeded inputs (float32; bf16-representable where the case is
bf16) and the expected outputs.  Re-run to regenerate:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import inputs as I  # noqa: E402
from oracle import mamba3_ref as M  # noqa: E402

SCAN_CASES = {
    # name: (B, L, H, N, P, R, CS, bf16, seed)
    "scan_f32_ref_unit_shape": (1, 70, 2, 64, 16, 16, 16, False, 101),
    "scan_f32_config1_geometry": (1, 130, 2, 64, 64, 16, 64, False, 102),
    "scan_bf16_headline_geometry": (1, 150, 2, 128, 64, 32, 64, True, 103),
}


def scan_case(B, L, H, N, P, R, CS, bf16, seed):
    d = I.scan_inputs(B, L, H, N, P, R, seed=seed, bf16=bf16)
    y = M.mamba3_ssd_chunked_batched(d["Q"], d["K"], d["V"], d["ADT"], d["DT"], d["Trap"],
                                      d["Angles"], d["Q_bias"], d["K_bias"], d["D"], d["Z"],
                                      chunk_size=CS)
    return dict(**d, Y=y, dims=np.array([B, L, H, N, P, R, CS, int(bf16)]))


def decode_case(B=2, H=2, N=128, P=64, R=32, steps=3, seed=104):
    d = I.decode_inputs(B, H, N, P, R, steps, seed=seed, bf16=True)
    carry = tuple(d[k].astype(np.float64) for k in ("theta", "h", "k_prev", "v_prev"))
    ys = []
    for s in range(steps):
        carry, y = M.rnn_step(carry, tuple(d[k][s] for k in ("x", "z", "Bt", "Ct", "adt", "dt",
                                                              "trap", "ang")),
                              d["B_bias"], d["C_bias"], d["D"])
        ys.append(y)
    return dict(**d, Y=np.stack(ys), theta_out=carry[0], h_out=carry[1], k_out=carry[2],
                v_out=carry[3], dims=np.array([B, H, N, P, R, steps]))


def main():
    for name, args in SCAN_CASES.items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **scan_case(*args))
    np.savez_compressed(os.path.join(HERE, "decode_bf16_headline_geometry.npz"), **decode_case())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
