"""Generate tests/golden/stack_config5_L12288.npz: the oracle backbone's per-token
log-probabilities for BASELINE configuration 5 at its full size, one batch row.

Configuration 5: the 12-layer Mamba3 backbone (d_model 768, expand 2, headdim 64,
d_state 128, half_glu1, prenorm, bf16 rounding points), vocabulary 2112, sequence
length 24 x 512 = 12288, random-init parameters (oracle.mamba3_stack.init_params,
seed 5) and token ids drawn uniformly from the vocabulary (numpy default_rng(505)).
The oracle (oracle/mamba3_stack.py, float64 over the pinned scan oracle) takes about
8 minutes here, too long for the GPU test run, so its output is kept as a fixture:
  positions  (64,)        int32   token positions spread over the sequence (the last included)
  logp_at    (64, 2112)   float32 log-probabilities at those positions
  argmax     (12288,)     int16   the most likely token at every position
  logp_max   (12288,)     float32 its log-probability
The GPU test rebuilds the same parameters and ids from the seeds.
    python tests/golden/make_golden_config5.py
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import mamba3_stack as MS  # noqa: E402

VOCAB, D_MODEL, LAYERS, L = 2112, 768, 12, 24 * 512
PARAM_SEED, IDS_SEED = 5, 505
N_POSITIONS = 64


def ids():
    return np.random.default_rng(IDS_SEED).integers(0, VOCAB, size=(1, L))


def positions():
    return np.linspace(0, L - 1, N_POSITIONS).round().astype(np.int32)


def main():
    t0 = time.time()
    p = MS.init_params(vocab=VOCAB, d_model=D_MODEL, n_layers=LAYERS, seed=PARAM_SEED)
    ref = MS.lm_forward(p, ids(), bf16=True)[0]
    pos = positions()
    am = ref.argmax(-1)
    out = dict(positions=pos, logp_at=ref[pos].astype(np.float32), argmax=am.astype(np.int16),
               logp_max=ref[np.arange(L), am].astype(np.float32))
    path = os.path.join(HERE, "stack_config5_L12288.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} in {time.time() - t0:.0f} s")


if __name__ == "__main__":
    main()
