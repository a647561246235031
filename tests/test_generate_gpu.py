"""Generation through the layer and the backbone: prefill with the recurrent carry,
then one token at a time (Mamba3SSM.__call_rnn__, mamba3.py:466-568).

Chunked == recurrent is the reference's own contract for the scan
(test_backbone_contracts.py:81-111, rtol 2e-5): a prefill of the first L0 tokens
followed by decode steps must give the outputs of the forward over the whole
sequence at the later positions, and so must a prefill in two pieces.  Bars: float32
1e-4 and bf16 2e-2 relative in norm (the forward's own bars against the oracle; the
decode step computes in float32 from bf16 operands where the chunked kernel rounds
its MFMA operands to bf16).  The prefill's own output equals the forward's bitwise in
bf16 (observed on both routes); in float32 the carry-writing kernel differs from the
plain one at rounding level (1.2e-7 observed, bar 1e-6).  The last test runs the
shape bench.py's generation line times (config 5's backbone, 512 sequences).
"""
import numpy as np
import pytest

from _util import rel
from oracle import mamba3_layer as ML
from oracle import mamba3_stack as MS

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,L0,S,d_model,N,hd,bf16,path", [
    (2, 150, 20, 256, 128, 64, True, "in_place"),     # 1336-wide bf16 rows
    (2, 150, 20, 128, 128, 64, True, "copies"),       # 812-wide bf16 rows: x and z copied
    (2, 150, 20, 64, 64, 32, False, "in_place"),      # float32, 412-wide rows
    (1, 1100, 12, 256, 128, 64, True, "in_place"),    # 8 pairs: the prefill takes the sequence split
])
def test_layer_prefill_then_decode_matches_forward(B, L0, S, d_model, N, hd, bf16, path):
    import torch
    from mamba3_rocm import Mamba3Layer
    dt = torch.bfloat16 if bf16 else torch.float32
    p = ML.init_params(d_model, seed=91, d_state=N, headdim=hd)
    layer = Mamba3Layer({k: torch.from_numpy(v).cuda() for k, v in p.items()}, d_model, d_state=N, headdim=hd,
                        dtype=dt)
    x = torch.from_numpy(np.random.default_rng(92).standard_normal((B, L0 + S, d_model)).astype(np.float32)).cuda()
    print(f"case layer generate {(B, L0, S, d_model, N, hd)} bf16={bf16} {path}", flush=True)
    full = layer(x)
    assert layer.last_scan == path
    out0, carry = layer.prefill(x[:, :L0].contiguous())
    assert layer.last_scan == path
    e_pre = rel(out0.float().cpu().numpy(), full[:, :L0].float().cpu().numpy())
    print(f"layer generate: prefill against the forward {e_pre:.2e} (bitwise: {torch.equal(out0, full[:, :L0])})",
          flush=True)
    if path == "in_place" and bf16:
        assert torch.equal(out0, full[:, :L0]), "prefill output differs from the forward's"
    else:
        assert e_pre <= 1e-6
    # a prefill in two pieces
    h = L0 // 2 + 3
    _, c1 = layer.prefill(x[:, :h].contiguous())
    o2, _ = layer.prefill(x[:, h:L0].contiguous(), c1)
    bar = 2e-2 if bf16 else 1e-4
    e_two = rel(o2.float().cpu().numpy(), full[:, h:L0].float().cpu().numpy())
    # decode steps after the prefill
    outs = []
    for t in range(S):
        o, carry = layer.step(x[:, L0 + t].contiguous(), carry)
        outs.append(o)
    torch.cuda.synchronize()
    dec = torch.stack(outs, 1).float().cpu().numpy()
    e_dec = rel(dec, full[:, L0:].float().cpu().numpy())
    print(f"layer generate: two-piece prefill {e_two:.2e}, decode {e_dec:.2e}", flush=True)
    assert e_two <= bar and e_dec <= bar


@pytest.mark.parametrize("bf16,activation,prenorm", [
    (False, "half_glu1", True), (True, "half_glu1", True),       # the LOB models' block
    (False, "full_glu", False), (True, "half_glu2", False),      # postnorm: the LayerNorm on the residual
    (False, "gelu", True),
])
def test_stack_prefill_then_decode_matches_logits(bf16, activation, prenorm):
    import torch
    from mamba3_rocm import Mamba3Stack
    N, hd, D, V = (128, 64, 128, 53) if bf16 else (64, 32, 64, 37)
    p = MS.init_params(vocab=V, d_model=D, n_layers=2, seed=93, d_state=N, headdim=hd)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()   # noqa: E731
    tp = dict(embed=t(p["embed"]), decoder_w=t(p["decoder_w"]), decoder_b=t(p["decoder_b"]),
              layers=[{k: ({kk: t(vv) for kk, vv in v.items()} if k == "mixer" else t(v)) for k, v in lp.items()}
                      for lp in p["layers"]])
    stack = Mamba3Stack(tp, D, activation=activation, prenorm=prenorm, d_state=N, headdim=hd,
                        dtype=torch.bfloat16 if bf16 else torch.float32)
    B, L0, S = 2, 140, 16
    ids = torch.from_numpy(np.random.default_rng(94).integers(0, V, size=(B, L0 + S))).cuda()
    print(f"case stack generate bf16={bf16} {activation} prenorm={prenorm}", flush=True)
    full = stack.logits(ids)
    lp0, state = stack.prefill(ids[:, :L0])
    assert rel(lp0.cpu().numpy(), full[:, :L0].cpu().numpy()) <= 1e-6
    outs = []
    for i in range(S):
        lpt, state = stack.step(ids[:, L0 + i], state)
        outs.append(lpt)
    torch.cuda.synchronize()
    dec = torch.stack(outs, 1).cpu().numpy()
    err = rel(dec, full[:, L0:].cpu().numpy())
    print(f"stack generate bf16={bf16} {activation} prenorm={prenorm}: decode log-probabilities {err:.2e}",
          flush=True)
    assert err <= (2e-2 if bf16 else 1e-4)


def test_stack_generation_at_the_bench_shape():
    """Config 5's backbone as bench.py's generation line runs it: 12 layers, d_model
    768, 24 heads, vocab 2112, 512 sequences, a 64-token prefill, then decode steps;
    every step's log-probabilities against the forward's logits over the whole
    sequence (the same bars as above)."""
    import torch
    from mamba3_rocm import Mamba3Stack
    from mamba3_rocm.stack import init_params
    B, L0, S, V = 512, 64, 8, 2112
    stack = Mamba3Stack(init_params(V, 768, 12, 95, "cuda"), 768, activation="half_glu1", prenorm=True,
                        dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(96)
    ids = torch.randint(0, V, (B, L0 + S), device="cuda", generator=g)
    print("case stack generate config 5, B=512", flush=True)
    full = stack.logits(ids)
    lp0, state = stack.prefill(ids[:, :L0])
    e_pre = rel(lp0.cpu().numpy(), full[:, :L0].cpu().numpy())
    outs = []
    for i in range(S):
        lpt, state = stack.step(ids[:, L0 + i].contiguous(), state)
        outs.append(lpt)
    torch.cuda.synchronize()
    dec = torch.stack(outs, 1).cpu().numpy()
    ref = full[:, L0:].cpu().numpy()
    err = rel(dec, ref)
    agree = float(np.mean(dec.argmax(-1) == ref.argmax(-1)))
    print(f"stack generate config 5: prefill {e_pre:.2e}, decode {err:.2e}, argmax agreement {agree:.4f}", flush=True)
    assert e_pre <= 1e-6
    assert err <= 2e-2


@pytest.mark.parametrize("bf16", [False, True])
def test_stack_step_graph_matches_eager_steps(bf16):
    """Mamba3Stack.step_graph: the step captured once in a HIP graph and replayed.
    Every replay against an eager step from a copy of the same carries, with eager work
    and a synchronisation between the replays (graph nodes that hold stale values show
    on the replays after the first); log-probabilities and carries to 1e-6 relative
    (the same kernels in the same order: bitwise equal is what is expected)."""
    import torch
    from mamba3_rocm import Mamba3Stack
    N, hd, D, V = (128, 64, 128, 53) if bf16 else (64, 32, 64, 37)
    p = MS.init_params(vocab=V, d_model=D, n_layers=2, seed=97, d_state=N, headdim=hd)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()   # noqa: E731
    tp = dict(embed=t(p["embed"]), decoder_w=t(p["decoder_w"]), decoder_b=t(p["decoder_b"]),
              layers=[{k: ({kk: t(vv) for kk, vv in v.items()} if k == "mixer" else t(v)) for k, v in lp.items()}
                      for lp in p["layers"]])
    stack = Mamba3Stack(tp, D, activation="half_glu1", prenorm=True, d_state=N, headdim=hd,
                        dtype=torch.bfloat16 if bf16 else torch.float32)
    B, L0, S = 3, 70, 6
    ids = torch.from_numpy(np.random.default_rng(98).integers(0, V, size=(B, L0 + S))).cuda()
    print(f"case stack step graph bf16={bf16}", flush=True)
    _, st_e = stack.prefill(ids[:, :L0])
    st_g = [tuple(x.clone() for x in c) for c in st_e]
    graph = stack.step_graph(st_g)
    worst, same = 0.0, True
    for i in range(S):
        lp_g = graph(ids[:, L0 + i]).clone()
        lp_e, _ = stack.step(ids[:, L0 + i].contiguous(), st_e)
        torch.cuda.synchronize()
        same = same and torch.equal(lp_g, lp_e)
        worst = max(worst, rel(lp_g.cpu().numpy(), lp_e.cpu().numpy()))
    for ce, cg in zip(st_e, st_g):
        for a, b in zip(ce, cg):
            same = same and torch.equal(a, b)
            worst = max(worst, rel(b.cpu().numpy(), a.cpu().numpy()))
    print(f"stack step graph bf16={bf16}: worst {worst:.2e}, bitwise {same}", flush=True)
    assert worst <= 1e-6
