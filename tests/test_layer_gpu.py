"""The Mamba3 mixer layer on the GPU vs the layer oracle (oracle/mamba3_layer.py).

Same parameters and input on both sides.  Bars: fp32 1e-4 (the scan's fp32 bar);
bf16 2e-2 (the scan's bf16 bar; the oracle rounds to bf16 where the reference's
bf16 layer does).  The reference's own bf16-vs-f32 layer bound is 5e-2
(test_mamba3_mixed_precision.py:86-104).
"""
import numpy as np
import pytest

from _util import rel
from oracle import mamba3_layer as ML

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,L,d_model,N,headdim,bf16", [
    (2, 200, 128, 128, 64, True),      # model geometry per head (d_state 128, headdim 64, 4 heads)
    (1, 1100, 64, 128, 64, True),      # B*H small: the scan's sequence split
    (2, 150, 64, 64, 32, False),       # fp32: chunked kernel shapes
])
def test_layer_matches_oracle(B, L, d_model, N, headdim, bf16):
    import torch
    from mamba3_rocm import Mamba3Layer
    p = ML.init_params(d_model, seed=51, d_state=N, headdim=headdim)
    x = np.random.default_rng(52).standard_normal((B, L, d_model)).astype(np.float32)
    dt = torch.bfloat16 if bf16 else torch.float32
    layer = Mamba3Layer({k: torch.from_numpy(v).cuda() for k, v in p.items()}, d_model, d_state=N,
                        headdim=headdim, dtype=dt)
    y = layer(torch.from_numpy(x).cuda()).float().cpu().numpy()
    ref = ML.layer_forward(p, x, d_state=N, headdim=headdim, bf16=bf16)
    err = rel(y, ref)
    print(f"layer {(B, L, d_model, N, headdim)} bf16={bf16} rel={err:.3e}", flush=True)
    assert np.isfinite(y).all()
    assert err <= (2e-2 if bf16 else 1e-4)
