"""Parity at the BASELINE configurations' own sizes (the other GPU tests use shapes
that the float64 oracle finishes quickly).

* Configuration 3, B=1, L=32768, H=32, chunk 128: the prefill takes the sequence
  split (8 segments of 4096 tokens).  Four heads over all 32768 tokens against the
  float64 oracle (bf16 bar 2e-2), and the split against one pass over the whole
  output.
* The backward at configuration 2's length, L=4096 (and 5120), on two heads: every
  gradient against autograd of the float64 oracle (bf16 bar 2e-2, tighter than the
  suite's 3e-2 for bf16 gradients: the whole-sequence cumsums behind dADT, dDT and
  dAngles are the ones that lose precision with length; float32 I/O at the model's
  geometry, the suite's 2e-5).
* The backward at configuration 3's shape (the split walk): two heads over all
  32768 tokens against the float64 oracle, and every head against the
  chunk-parallel route (2e-2; 5e-2 for the whole-sequence cumsums dAngles and dADT,
  whose bf16 rounding grows with the length).
* The backward at configuration 2's full shape (B=8, L=4096, H=32: the walk on all
  256 workgroups at once): two (batch, head) pairs against the float64 oracle, every
  gradient against the chunk-parallel route, and the training pair's backward equal to
  the recomputing one bitwise.
* The backward at configuration 5's layer shape (B=4, L=12288, H=24: 96 pairs, the
  split walk in 8 segments): two pairs against the float64 oracle, every gradient
  against the one-segment walk (the bars of configuration 3's shape), and the
  training pair's backward equal to the recomputing one bitwise.
* Configuration 5, the 12-layer backbone at L=12288: batch row 0 against the oracle
  backbone's log-probabilities (a committed fixture, tests/golden/
  make_golden_config5.py: the oracle takes minutes at this size): 64 positions within
  2e-2, and the most likely token at every position; all four rows finite.
"""
import os

import numpy as np
import pytest

from _util import I, M, device_scan_inputs, heads_to_numpy, rel

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
GRAD_TOL = 2e-2
F32_GRAD_TOL = 2e-5
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.timeout(300)
def test_config3_full_size_split_matches_oracle_and_one_pass():
    import torch
    from mamba3_rocm import _lib, mamba3_siso_hip
    B, L, H, N, P, R, CS = 1, 32768, 32, 128, 64, 32, 128
    assert _lib.load().m3_chunk_scan_ws_bytes(B, L, H, N, P, R, CS, _lib.DTYPE_BF16) > 0, "config 3 splits"
    print(f"[sizes] config 3 {(B, L, H, N, P, R, CS)}", flush=True)
    t = device_scan_inputs(B, L, H, N, P, R, seed=3, io_dtype=torch.bfloat16)
    args = [t[k] for k in ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")]
    split = mamba3_siso_hip(*args, chunk_size=CS)
    one = mamba3_siso_hip(*args, chunk_size=CS, seq_split=False)
    torch.cuda.synchronize()
    assert torch.isfinite(split.float()).all()
    e_one = rel(split.float().cpu().numpy(), one.float().cpu().numpy())
    heads = [0, 9, 21, 31]
    d = heads_to_numpy(t, heads)
    ref = M.mamba3_ssd_chunked_batched(d["Q"], d["K"], d["V"], d["ADT"], d["DT"], d["Trap"], d["Angles"],
                                       d["Q_bias"], d["K_bias"], d["D"], d["Z"], chunk_size=CS)
    e = rel(split[:, :, heads].float().cpu().numpy(), ref)
    print(f"  split vs oracle (heads {heads}, all {L} tokens): {e:.3e}; split vs one pass: {e_one:.3e}",
          flush=True)
    assert e <= BF16_TOL
    assert e_one <= 1e-2


@pytest.mark.timeout(300)
@pytest.mark.parametrize("L,bf16", [(4096, True), (5120, True), (4096, False)])
def test_backward_at_config2_length(L, bf16, bwd_route):
    import torch
    from mamba3_rocm import mamba3_siso_hip_bwd
    from oracle import mamba3_vjp as V
    B, H, N, P, R, CS = 1, 2, 128, 64, 32, 64
    print(f"[sizes] backward {(B, L, H, N, P, R, CS)} bf16={bf16} route={bwd_route}", flush=True)
    d = I.scan_inputs(B, L, H, N, P, R, seed=38, bf16=bf16)
    cot = V.cotangent(B, L, H, P, seed=39)
    if bf16:
        cot = I.bf16_round(cot)
    io = torch.bfloat16 if bf16 else torch.float32
    t = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in d.items()}
    for k in ("Q", "K", "V", "Z"):
        t[k] = t[k].to(io)
    dout = torch.from_numpy(np.ascontiguousarray(cot)).cuda().to(io)
    got = mamba3_siso_hip_bwd(*(t[k] for k in V.NAMES), dout, chunk_size=CS)
    torch.cuda.synchronize()
    _, ref = V.vjp(d, cot, CS)
    errs = {}
    for name, a, b in zip(V.NAMES, got, ref):
        a = a.float().cpu().numpy()
        assert np.isfinite(a).all(), name
        errs[name] = rel(a, b)
    print("  " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    tol = GRAD_TOL if bf16 else F32_GRAD_TOL
    bad = {k: v for k, v in errs.items() if v > tol}
    assert not bad, f"gradients above {tol}: {bad}"


@pytest.mark.timeout(300)
def test_backward_config3_full_size_split_walk(monkeypatch):
    """The backward at configuration 3's shape (B=1, L=32768, H=32: 32 pairs, so the
    walk is split into 8 segments of 64 chunks and the state pass into 8 segments of
    4096 tokens): two heads' eleven gradients over all 32768 tokens against autograd of
    the float64 oracle, and every gradient of every head against the chunk-parallel
    route, which shares no segment algebra with it."""
    import torch
    from mamba3_rocm import mamba3_siso_hip_bwd
    from oracle import mamba3_vjp as V
    B, L, H, N, P, R, CS = 1, 32768, 32, 128, 64, 32, 128
    print(f"[sizes] backward config 3 {(B, L, H, N, P, R, CS)} split walk", flush=True)
    monkeypatch.delenv("M3_BWD_ROUTE", raising=False)
    t = device_scan_inputs(B, L, H, N, P, R, seed=40, io_dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(41)
    dout = torch.randn(B, L, H, P, device="cuda", generator=g).to(torch.bfloat16)
    args = tuple(t[k] for k in V.NAMES)
    got = mamba3_siso_hip_bwd(*args, dout, chunk_size=CS)
    monkeypatch.setenv("M3_BWD_ROUTE", "chunks")
    alt = mamba3_siso_hip_bwd(*args, dout, chunk_size=CS)
    torch.cuda.synchronize()
    e_alt = {k: rel(a.float().cpu().numpy(), b.float().cpu().numpy()) for k, a, b in zip(V.NAMES, got, alt)}
    print("  split walk vs chunk route: " + " ".join(f"{k}:{v:.1e}" for k, v in e_alt.items()), flush=True)
    heads = [0, 17]
    d = heads_to_numpy(t, heads)
    cot = dout.index_select(2, torch.as_tensor(heads, device="cuda")).float().cpu().numpy()
    _, ref = V.vjp(d, cot, 64)
    hsel = torch.as_tensor(heads, device="cuda")
    errs = {}
    for name, a, r in zip(V.NAMES, got, ref):
        dim = {"Q": 2, "K": 2, "V": 2, "Z": 2, "Angles": 2, "ADT": 1, "DT": 1, "Trap": 1}.get(name, 0)
        a = a.index_select(dim, hsel).float().cpu().numpy()
        assert np.isfinite(a).all(), name
        errs[name] = rel(a, r)
    print(f"  heads {heads} vs oracle: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    # dAngles and dADT are reverse cumsums over the whole sequence, whose bf16 rounding
    # grows with the length (at L=4096 about 1.2e-2, here about 3e-2, on either route):
    # 5e-2 for them, half the reference's bf16 gradient bar (1e-1,
    # tests/integration/test_mamba3_pallas_gpu.py:66-69); 2e-2 for the others
    bar = lambda k: 5e-2 if k in ("Angles", "ADT") else GRAD_TOL  # noqa: E731
    bad = {k: v for k, v in errs.items() if v > bar(k)}
    assert not bad, f"gradients above their bar: {bad}"
    bad = {k: v for k, v in e_alt.items() if v > bar(k)}
    assert not bad, f"split walk and chunk route differ: {bad}"



@pytest.mark.timeout(300)
def test_backward_config2_full_size_walk(monkeypatch):
    """The backward at configuration 2's own shape (B=8, L=4096, H=32; 256 pairs, so the
    walk runs unsplit on every workgroup at once, the bench's configuration): pairs
    (b, h) = (0, 0) and (5, 19) against autograd of the float64 oracle on their own
    problem; every gradient of every pair against the chunk-parallel route (no shared
    code with the walk beyond the state pass); the training pair's backward (the saved
    chunk states instead of the state pass) equal to the recomputing one bitwise."""
    import torch
    from mamba3_rocm import mamba3_siso_hip_bwd, mamba3_siso_hip_fwd_train
    from oracle import mamba3_vjp as V
    B, L, H, N, P, R, CS = 8, 4096, 32, 128, 64, 32, 64
    print(f"[sizes] backward config 2 {(B, L, H, N, P, R, CS)} walk", flush=True)
    monkeypatch.delenv("M3_BWD_ROUTE", raising=False)
    t = device_scan_inputs(B, L, H, N, P, R, seed=42, io_dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(43)
    dout = torch.randn(B, L, H, P, device="cuda", generator=g).to(torch.bfloat16)
    args = tuple(t[k] for k in V.NAMES)
    got = mamba3_siso_hip_bwd(*args, dout, chunk_size=CS)
    _, saved = mamba3_siso_hip_fwd_train(*args, chunk_size=CS)
    from_saved = mamba3_siso_hip_bwd(*args, dout, chunk_size=CS, saved=saved)
    monkeypatch.setenv("M3_BWD_ROUTE", "chunks")
    alt = mamba3_siso_hip_bwd(*args, dout, chunk_size=CS)
    torch.cuda.synchronize()
    for k, a, b in zip(V.NAMES, got, from_saved):
        assert torch.equal(a, b), f"training pair differs from the recomputing backward in d{k}"
    e_alt = {k: rel(a.float().cpu().numpy(), b.float().cpu().numpy()) for k, a, b in zip(V.NAMES, got, alt)}
    print("  walk vs chunk route: " + " ".join(f"{k}:{v:.1e}" for k, v in e_alt.items()), flush=True)
    # per-(b, h) inputs and gradients: batch and head axes of each tensor (biases and D
    # are per head, their gradients summed over the batch: checked against the chunk
    # route only)
    axes = {"Q": (0, 2), "K": (0, 2), "V": (0, 2), "Z": (0, 2), "Angles": (0, 2), "ADT": (0, 1), "DT": (0, 1),
            "Trap": (0, 1), "Q_bias": (None, 0), "K_bias": (None, 0), "D": (None, 0)}
    def pick(x, name, b, h):
        ba, ha = axes[name]
        x = x.narrow(ha, h, 1)
        return x.narrow(ba, b, 1) if ba is not None else x
    for b, h in ((0, 0), (5, 19)):
        d = {k: pick(t[k], k, b, h).float().cpu().numpy() for k in V.NAMES}
        cot = dout[b:b + 1, :, h:h + 1].float().cpu().numpy()
        _, ref = V.vjp(d, cot, CS)
        errs = {}
        for name, a, r in zip(V.NAMES, got, ref):
            if axes[name][0] is None:
                continue
            a = pick(a, name, b, h).float().cpu().numpy()
            assert np.isfinite(a).all(), name
            errs[name] = rel(a, r)
        print(f"  pair {(b, h)} vs oracle: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
        bad = {k: v for k, v in errs.items() if v > GRAD_TOL}
        assert not bad, f"pair {(b, h)}: gradients above {GRAD_TOL}: {bad}"
    bad = {k: v for k, v in e_alt.items() if v > GRAD_TOL}
    assert not bad, f"walk and chunk route differ: {bad}"


@pytest.mark.timeout(300)
def test_backward_config5_layer_shape_split_walk(monkeypatch):
    """The backward at configuration 5's layer shape (B=4, L=12288, H=24: 96 pairs, so
    the walk is split into 8 segments of 24 chunks, three rounds of 256 workgroups, and
    its state pass into the forward's 8-segment split): pairs (b, h) = (0, 0) and
    (3, 17) against autograd of the float64 oracle on their own problem; every
    gradient of every pair against the one-segment walk; the training pair's backward
    equal to the recomputing one bitwise."""
    import torch
    from mamba3_rocm import mamba3_siso_hip_bwd, mamba3_siso_hip_fwd_train
    from oracle import mamba3_vjp as V
    B, L, H, N, P, R, CS = 4, 12288, 24, 128, 64, 32, 64
    print(f"[sizes] backward config 5 layer {(B, L, H, N, P, R, CS)} split walk", flush=True)
    monkeypatch.delenv("M3_BWD_ROUTE", raising=False)
    t = device_scan_inputs(B, L, H, N, P, R, seed=52, io_dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(53)
    dout = torch.randn(B, L, H, P, device="cuda", generator=g).to(torch.bfloat16)
    args = tuple(t[k] for k in V.NAMES)
    got = mamba3_siso_hip_bwd(*args, dout, chunk_size=CS)
    _, saved = mamba3_siso_hip_fwd_train(*args, chunk_size=CS)
    from_saved = mamba3_siso_hip_bwd(*args, dout, chunk_size=CS, saved=saved)
    monkeypatch.setenv("M3_BWD_ROUTE", "walk")
    alt = mamba3_siso_hip_bwd(*args, dout, chunk_size=CS)
    torch.cuda.synchronize()
    for k, a, b in zip(V.NAMES, got, from_saved):
        assert torch.equal(a, b), f"training pair differs from the recomputing backward in d{k}"
    e_alt = {k: rel(a.float().cpu().numpy(), b.float().cpu().numpy()) for k, a, b in zip(V.NAMES, got, alt)}
    print("  split vs one-segment walk: " + " ".join(f"{k}:{v:.1e}" for k, v in e_alt.items()), flush=True)
    # the whole-sequence reverse cumsums dAngles and dADT lose precision with the length
    # as at config 3's shape: 5e-2 for them, 2e-2 for the others
    bar = lambda k: 5e-2 if k in ("Angles", "ADT") else GRAD_TOL  # noqa: E731
    axes = {"Q": (0, 2), "K": (0, 2), "V": (0, 2), "Z": (0, 2), "Angles": (0, 2), "ADT": (0, 1), "DT": (0, 1),
            "Trap": (0, 1), "Q_bias": (None, 0), "K_bias": (None, 0), "D": (None, 0)}
    def pick(x, name, b, h):
        ba, ha = axes[name]
        x = x.narrow(ha, h, 1)
        return x.narrow(ba, b, 1) if ba is not None else x
    for b, h in ((0, 0), (3, 17)):
        d = {k: pick(t[k], k, b, h).float().cpu().numpy() for k in V.NAMES}
        cot = dout[b:b + 1, :, h:h + 1].float().cpu().numpy()
        _, ref = V.vjp(d, cot, CS)
        errs = {}
        for name, a, r in zip(V.NAMES, got, ref):
            if axes[name][0] is None:
                continue
            a = pick(a, name, b, h).float().cpu().numpy()
            assert np.isfinite(a).all(), name
            errs[name] = rel(a, r)
        print(f"  pair {(b, h)} vs oracle: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
        bad = {k: v for k, v in errs.items() if v > bar(k)}
        assert not bad, f"pair {(b, h)}: gradients above their bar: {bad}"
    bad = {k: v for k, v in e_alt.items() if v > bar(k)}
    assert not bad, f"split and one-segment walk differ: {bad}"


def _torch_params(p):
    import torch
    cuda = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    return dict(embed=cuda(p["embed"]), decoder_w=cuda(p["decoder_w"]), decoder_b=cuda(p["decoder_b"]),
                layers=[{k: ({kk: cuda(vv) for kk, vv in v.items()} if k == "mixer" else cuda(v))
                         for k, v in lp.items()} for lp in p["layers"]])


@pytest.mark.timeout(300)
def test_config5_backbone_full_size_matches_oracle_fixture():
    import sys
    import torch
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import make_golden_config5 as G
    from mamba3_rocm import Mamba3Stack
    from oracle import mamba3_stack as MS
    fx = np.load(os.path.join(HERE, "golden", "stack_config5_L12288.npz"))
    p = MS.init_params(vocab=G.VOCAB, d_model=G.D_MODEL, n_layers=G.LAYERS, seed=G.PARAM_SEED)
    ids0 = G.ids()
    others = np.random.default_rng(506).integers(0, G.VOCAB, size=(3, G.L))
    ids = torch.from_numpy(np.concatenate([ids0, others])).cuda()          # B = 4, row 0 checked
    print(f"[sizes] config 5 backbone B=4 L={G.L} layers={G.LAYERS}", flush=True)
    stack = Mamba3Stack(_torch_params(p), G.D_MODEL, activation="half_glu1", prenorm=True, dtype=torch.bfloat16)
    lp = stack.logits(ids)
    torch.cuda.synchronize()
    assert lp.shape == (4, G.L, G.VOCAB) and lp.dtype == torch.float32
    assert torch.isfinite(lp).all()
    assert stack.blocks[0]["mixer"].last_scan == "in_place", "config 5 reads x and z in place"
    got = lp[0].cpu().numpy()
    pos = fx["positions"]
    e = rel(got[pos], fx["logp_at"])
    am = got.argmax(-1)
    agree = float(np.mean(am == fx["argmax"]))
    # where the most likely tokens differ, the oracle's choice is a near tie
    gap = float(np.abs(got[np.arange(G.L), fx["argmax"].astype(np.int64)] - fx["logp_max"]).max())
    print(f"  row 0: log-probabilities at {len(pos)} positions rel {e:.3e}; argmax agreement {agree:.4f}; "
          f"max |logp at the oracle's argmax - oracle| {gap:.3e}", flush=True)
    assert e <= BF16_TOL
    assert agree >= 0.98
    assert gap <= BF16_TOL * np.abs(fx["logp_at"]).max()
    # every position of every row: the bf16 backbone against the same backbone computed
    # in float32 (the float32 path that the oracle pins at 1e-4 at smaller sizes), all
    # 4 x 12288 x 2112 log-probabilities
    s32 = Mamba3Stack(_torch_params(p), G.D_MODEL, activation="half_glu1", prenorm=True, dtype=torch.float32)
    lp32 = s32.logits(ids)
    torch.cuda.synchronize()
    e_all = float((lp - lp32).norm() / lp32.norm())
    agree_all = float((lp.argmax(-1) == lp32.argmax(-1)).float().mean())
    print(f"  all rows, every position: bf16 against float32 rel {e_all:.3e}; argmax agreement {agree_all:.4f}",
          flush=True)
    assert e_all <= BF16_TOL
    assert agree_all >= 0.98
