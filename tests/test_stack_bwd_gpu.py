"""The backbone's training step (Mamba3Stack.loss_and_grads).

* float32 compute against central finite differences of the float64 stack oracle
  (oracle/mamba3_stack.py lm_forward): the loss is the mean negative log-likelihood
  of target tokens; for each tested parameter a random direction u of its shape, and
  the directional derivative <grad, u> against (f(p + e u) - f(p - e u)) / 2e, bar
  1e-3 (the float32 layer backward meets 2.2e-4 against the same kind of quotient).
  e = 1e-5 of the parameter's scale: the quotient's truncation error falls as e^2
  (the decoder kernel's direction, whose derivative is small against the gradient's
  norm, differs from the oracle's closed form featuresᵀ (softmax - onehot) / n by
  1.7e-2, 1.7e-4 and 1.6e-6 at e = 1e-3, 1e-4, 1e-5), and the float64 oracle's
  rounding is far below it.  Parameters the activation leaves unused must get
  exactly zero.
* The loss itself against the oracle's, float32 bar 1e-4.
* bf16 compute against float32 of the same stack, every gradient within the
  reference's bf16 gradient bar of 1e-1 (tests/integration/test_mamba3_pallas_gpu.py:
  66-69), relative in norm.
"""
import copy

import numpy as np
import pytest

from _util import rel
from oracle import mamba3_stack as MS

pytestmark = pytest.mark.gpu


def _tp(p):
    import torch
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()   # noqa: E731
    return dict(embed=t(p["embed"]), decoder_w=t(p["decoder_w"]), decoder_b=t(p["decoder_b"]),
                layers=[{k: ({kk: t(vv) for kk, vv in v.items()} if k == "mixer" else t(v)) for k, v in lp.items()}
                        for lp in p["layers"]])


def _get(d, path):
    for k in path:
        d = d[k]
    return d


def _nll(p, ids, tg, activation, N, hd):
    lp = MS.lm_forward(p, ids, activation=activation, prenorm=True, d_state=N, headdim=hd)
    return -float(np.mean(np.take_along_axis(lp, tg[..., None], axis=-1)))


def _run(p, ids, tg, activation, D, N, hd, dtype):
    import torch
    from mamba3_rocm import Mamba3Stack
    stack = Mamba3Stack(_tp(p), D, activation=activation, prenorm=True, d_state=N, headdim=hd, dtype=dtype)
    loss, g = stack.loss_and_grads(torch.from_numpy(ids).cuda(), torch.from_numpy(tg).cuda())
    torch.cuda.synchronize()
    return float(loss), g


PATHS = [("embed",), ("decoder_w",), ("decoder_b",), ("layers", 0, "ln_scale"), ("layers", 0, "ln_bias"),
         ("layers", 1, "ln_scale"), ("layers", 0, "out2_w"), ("layers", 1, "out2_b"), ("layers", 0, "out1_w"),
         ("layers", 1, "out1_b"), ("layers", 0, "mixer", "in_proj"), ("layers", 1, "mixer", "dt_bias"),
         ("layers", 0, "mixer", "B_norm"), ("layers", 1, "mixer", "out_proj"), ("layers", 0, "mixer", "D")]


@pytest.mark.parametrize("activation", ["half_glu1", "full_glu", "half_glu2", "gelu"])
def test_stack_grads_f32_match_finite_differences(activation):
    import torch
    N, hd, V, D = 64, 32, 37, 64
    p = MS.init_params(vocab=V, d_model=D, n_layers=2, seed=81, d_state=N, headdim=hd)
    rng = np.random.default_rng(82)
    ids = rng.integers(0, V, size=(2, 150))
    tg = rng.integers(0, V, size=(2, 150))
    print(f"case stack grads f32 {activation}", flush=True)
    loss, g = _run(p, ids, tg, activation, D, N, hd, torch.float32)
    ref = _nll(p, ids, tg, activation, N, hd)
    assert abs(loss - ref) <= 1e-4 * abs(ref), (loss, ref)
    unused = {"out1_w", "out1_b"} if activation != "full_glu" else set()
    if activation == "gelu":
        unused |= {"out2_w", "out2_b"}
    errs = {}
    for i, path in enumerate(PATHS):
        grad = _get(g, path).float().cpu().numpy().astype(np.float64)
        base = _get(p, path)
        assert grad.shape == base.shape, path
        assert np.isfinite(grad).all(), path
        if path[-1] in unused:
            assert not grad.any(), f"{path}: unused by {activation}, gradient not zero"
            continue
        u = np.random.default_rng(200 + i).standard_normal(base.shape)
        e = 1e-5 * max(1.0, float(np.abs(base).max()))

        def at(sgn):
            pp = copy.deepcopy(p)
            tgt = _get(pp, path[:-1])
            tgt[path[-1]] = base + sgn * e * u
            return _nll(pp, ids, tg, activation, N, hd)
        fd = (at(1.0) - at(-1.0)) / (2.0 * e)
        an = float(np.sum(grad * u))
        errs["/".join(map(str, path))] = abs(an - fd) / max(abs(fd), 1e-12)
    print(f"stack grads f32 {activation}: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if v > 1e-3}
    assert not bad, f"directional derivatives above 1e-3: {bad}"


def test_stack_grads_bf16_match_f32():
    import torch
    N, hd, V, D = 128, 64, 53, 128
    p = MS.init_params(vocab=V, d_model=D, n_layers=2, seed=83, d_state=N, headdim=hd)
    rng = np.random.default_rng(84)
    ids = rng.integers(0, V, size=(2, 330))
    tg = rng.integers(0, V, size=(2, 330))
    print("case stack grads bf16 vs f32", flush=True)
    l32, g32 = _run(p, ids, tg, "half_glu1", D, N, hd, torch.float32)
    l16, g16 = _run(p, ids, tg, "half_glu1", D, N, hd, torch.bfloat16)
    assert abs(l16 - l32) <= 2e-2 * abs(l32), (l16, l32)
    errs = {}
    for path in PATHS:
        if path[-1] in ("out1_w", "out1_b"):
            continue
        a = _get(g16, path).float().cpu().numpy()
        b = _get(g32, path).float().cpu().numpy()
        errs["/".join(map(str, path))] = rel(a, b)
    for i in range(2):
        for k in ("in_proj", "dt_bias", "B_bias", "C_bias", "B_norm", "C_norm", "D", "out_norm", "out_proj"):
            errs[f"layers/{i}/mixer/{k}"] = rel(g16["layers"][i]["mixer"][k].float().cpu().numpy(),
                                                g32["layers"][i]["mixer"][k].float().cpu().numpy())
    print("stack grads bf16 vs f32: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if v > 1e-1}
    assert not bad, f"bf16 gradients above 1e-1 of the float32 ones: {bad}"
