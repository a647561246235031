"""The Mamba3 mixer layer on the GPU vs the layer oracle (oracle/mamba3_layer.py).

Same parameters and input on both sides.  Bars: fp32 1e-4 (the scan's fp32 bar);
bf16 2e-2 (the scan's bf16 bar; the oracle rounds to bf16 where the reference's
bf16 layer does).  The reference's own bf16-vs-f32 layer bound is 5e-2
(test_mamba3_mixed_precision.py:86-104).
"""
import math

import numpy as np
import pytest

from _util import rel
from oracle import mamba3_layer as ML

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,L,d_model,N,headdim,bf16,path,split", [
    (2, 200, 128, 128, 64, True, "copies", False),    # model geometry per head; 812-wide rows: x, z copied
    (2, 330, 256, 128, 64, True, "in_place", False),  # 1336-wide bf16 rows (16-byte multiple): read in place
    (1, 1100, 64, 128, 64, True, "copies", True),     # B*H small: the scan's sequence split
    (1, 1100, 256, 128, 64, True, "in_place", True),  # in place and split (config 5's route: strided V/Z
                                                      # offsets in the state-only and per-segment passes)
    (2, 150, 64, 64, 32, False, "in_place", False),   # fp32: chunked kernel shapes, 412-wide rows in place
    (1, 100, 1024, 256, 64, True, "copies", False),   # d_state 256: generic scan; layer_pre tiles of 32 tokens
])
def test_layer_matches_oracle(B, L, d_model, N, headdim, bf16, path, split):
    import torch
    from mamba3_rocm import Mamba3Layer, _lib
    H, R = 2 * d_model // headdim, N // 4
    io = _lib.DTYPE_BF16 if bf16 else _lib.DTYPE_F32
    assert (_lib.load().m3_chunk_scan_ws_bytes(B, L, H, N, headdim, R, 64, io) > 0) == split
    p = ML.init_params(d_model, seed=51, d_state=N, headdim=headdim)
    x = np.random.default_rng(52).standard_normal((B, L, d_model)).astype(np.float32)
    dt = torch.bfloat16 if bf16 else torch.float32
    layer = Mamba3Layer({k: torch.from_numpy(v).cuda() for k, v in p.items()}, d_model, d_state=N,
                        headdim=headdim, dtype=dt)
    y = layer(torch.from_numpy(x).cuda()).float().cpu().numpy()
    ref = ML.layer_forward(p, x, d_state=N, headdim=headdim, bf16=bf16)
    err = rel(y, ref)
    print(f"layer {(B, L, d_model, N, headdim)} bf16={bf16} {layer.last_scan} rel={err:.3e}", flush=True)
    assert layer.last_scan == path
    assert np.isfinite(y).all()
    assert err <= (2e-2 if bf16 else 1e-4)


@pytest.mark.parametrize("layer_bf16,knob", [(True, "float32"), (False, "bfloat16")])
def test_layer_honours_pallas_dtype_knob(layer_bf16, knob, monkeypatch):
    """MAMBA3_PALLAS_DTYPE (mamba3_pallas.py:112-122) sets the scan's operand dtype
    apart from the layer's: the layer copies x and z and hands the scan operands in
    the knob's dtype.  The output stays in the layer's dtype and follows the oracle
    of the layer's dtype within the bf16 bar (one side of the comparison rounds to
    bf16)."""
    import torch
    from mamba3_rocm import Mamba3Layer
    B, L, d_model, N, headdim = 2, 200, 256, 128, 64
    monkeypatch.setenv("MAMBA3_PALLAS_DTYPE", knob)
    p = ML.init_params(d_model, seed=53, d_state=N, headdim=headdim)
    x = np.random.default_rng(54).standard_normal((B, L, d_model)).astype(np.float32)
    dt = torch.bfloat16 if layer_bf16 else torch.float32
    layer = Mamba3Layer({k: torch.from_numpy(v).cuda() for k, v in p.items()}, d_model, d_state=N,
                        headdim=headdim, dtype=dt)
    y = layer(torch.from_numpy(x).cuda())
    assert y.dtype == dt
    assert layer.last_scan == "copies" and layer.last_compute_dtype == getattr(torch, knob)
    ref = ML.layer_forward(p, x, d_state=N, headdim=headdim, bf16=layer_bf16)
    err = rel(y.float().cpu().numpy(), ref)
    print(f"layer knob={knob} layer_bf16={layer_bf16} rel={err:.3e}", flush=True)
    assert err <= 2e-2


@pytest.mark.parametrize("activation,prenorm,bf16", [
    ("half_glu1", True, True), ("full_glu", False, True), ("half_glu2", True, False), ("gelu", False, False),
])
def test_stack_matches_oracle(activation, prenorm, bf16):
    """Embedding + two SequenceLayer blocks with the Mamba3 mixer vs the stack oracle."""
    import torch
    from mamba3_rocm import Mamba3Stack
    from oracle import mamba3_stack as MS
    N, hd = (128, 64) if bf16 else (64, 32)
    p = MS.init_params(vocab=37, d_model=64, n_layers=2, seed=61, d_state=N, headdim=hd)
    ids = np.random.default_rng(62).integers(0, 37, size=(2, 260))
    tp = dict(embed=torch.from_numpy(p["embed"]).cuda(), decoder_w=torch.from_numpy(p["decoder_w"]).cuda(),
              decoder_b=torch.from_numpy(p["decoder_b"]).cuda(), layers=[{k: ({kk: torch.from_numpy(vv).cuda() for kk, vv in v.items()} if k == "mixer"
                           else torch.from_numpy(v).cuda()) for k, v in lp.items()} for lp in p["layers"]])
    stack = Mamba3Stack(tp, 64, activation=activation, prenorm=prenorm, d_state=N, headdim=hd,
                        dtype=torch.bfloat16 if bf16 else torch.float32)
    y = stack(torch.from_numpy(ids).cuda()).float().cpu().numpy()
    ref = MS.stack_forward(p, ids, activation=activation, prenorm=prenorm, d_state=N, headdim=hd, bf16=bf16)
    err = rel(y, ref)
    print(f"stack {activation} prenorm={prenorm} bf16={bf16} rel={err:.3e}", flush=True)
    assert err <= (2e-2 if bf16 else 1e-4)


def _torch_params(p):
    import torch
    t = lambda a: torch.from_numpy(a).cuda()   # noqa: E731
    return dict(embed=t(p["embed"]), decoder_w=t(p["decoder_w"]), decoder_b=t(p["decoder_b"]),
                layers=[{k: ({kk: t(vv) for kk, vv in v.items()} if k == "mixer" else t(v))
                         for k, v in lp.items()} for lp in p["layers"]])


def test_backbone_logits_config5_geometry():
    """Config 5's model geometry (d_model 768, 24 heads of 64, d_state 128, vocab 2112,
    half_glu1, prenorm, bf16) with 2 of its 12 layers on a short sequence: per-token
    log-probabilities vs the oracle backbone, max-rel-err within 2e-2."""
    import torch
    from mamba3_rocm import Mamba3Stack
    from oracle import mamba3_stack as MS
    p = MS.init_params(vocab=2112, d_model=768, n_layers=2, seed=5)
    ids = np.random.default_rng(55).integers(0, 2112, size=(1, 200))
    stack = Mamba3Stack(_torch_params(p), 768, dtype=torch.bfloat16)
    lp = stack.logits(torch.from_numpy(ids).cuda()).cpu().numpy()
    ref = MS.lm_forward(p, ids, bf16=True)
    err = rel(lp, ref)
    agree = float(np.mean(np.argmax(lp, -1) == np.argmax(ref, -1)))
    print(f"stack logits config5 geometry rel={err:.3e} argmax agreement={agree:.4f}", flush=True)
    assert lp.dtype == np.float32 and err <= 2e-2


@pytest.mark.parametrize("B,L,D,bf16", [
    (2, 37, 768, True),     # config 5's width: the register path
    (1, 9, 100, False),     # fp32, D % 8 != 0: 16-byte norm rows, scalar elementwise path
    (1, 5, 2050, True),     # D > 2048 and D % 4 != 0: the norm's scalar path
])
def test_block_kernels_match_torch_fp32(B, L, D, bf16):
    """m3_block_norm / m3_block_gelu / m3_block_act against torch restatements of
    LayerNorm (float32, eps 1e-6), the tanh gelu and the four activation epilogues
    (float64, the oracle's precision, with the same rounding points).  fp32: 2e-6
    relative to the largest element; bf16: within 2^-7 relative per element (a last-bit
    difference in float32 can flip one rounding).  The gelu reference is float64
    is x * sigmoid(2u) in float64, equal to 0.5 x (1 + tanh(u)) (checked to 1e-12 where
    the latter is accurate): 1 + tanh(u) cancels for x below about -4.5 in float32 and
    about -7 in float64."""
    import torch
    import torch.nn.functional as F
    from mamba3_rocm import _lib
    from mamba3_rocm.ops import _stream
    lib = _lib.load()
    g = torch.Generator(device="cuda").manual_seed(71)
    dt = torch.bfloat16 if bf16 else torch.float32
    io = _lib.DTYPE_BF16 if bf16 else _lib.DTYPE_F32
    x = torch.randn(B, L, D, device="cuda", generator=g) * 3 + 0.5
    sc = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
    bi = 0.1 * torch.randn(D, device="cuda", generator=g)
    st = _stream(x)
    r = (lambda t: t.to(dt).double())         # noqa: E731

    def close(got, want, what):
        got, want = got.double(), want.double()
        if bf16:
            # absolute floor: below x = -10.7 exp(-2u) overflows float32 and the kernel's gelu
            # is -0 where the exact value is under 1e-38
            tol = want.abs() * 2 ** -7 * 1.01 + 1e-30
            bad = ((got - want).abs() > tol).sum().item()
            assert bad == 0, f"{what}: {bad} elements outside 2^-7 relative"
        else:
            err = ((got - want).abs().max() / want.abs().max()).item()
            assert err <= 2e-6, f"{what}: rel {err:.2e}"

    ln_ref = F.layer_norm(x, (D,), sc, bi, eps=1e-6)
    out = torch.empty(B, L, D, device="cuda", dtype=dt)
    _lib.check(lib.m3_block_norm(x.data_ptr(), sc.data_ptr(), bi.data_ptr(), out.data_ptr(), B, L, D, 1e-6, io, st),
               "m3_block_norm")
    close(out, r(ln_ref), "norm")
    o32 = x.clone()
    _lib.check(lib.m3_block_norm(o32.data_ptr(), sc.data_ptr(), bi.data_ptr(), o32.data_ptr(), B, L, D, 1e-6,
                                 _lib.DTYPE_F32, st), "m3_block_norm f32 in place")
    assert ((o32 - ln_ref).abs().max() / ln_ref.abs().max()).item() <= 2e-6

    y = r(x).to(dt).contiguous()
    gl = torch.empty_like(y)
    _lib.check(lib.m3_block_gelu(y.data_ptr(), gl.data_ptr(), B, L, D, io, st), "m3_block_gelu")
    yd = y.double()
    gelu_ref = yd * torch.sigmoid(2 * math.sqrt(2 / math.pi) * (yd + 0.044715 * yd ** 3))
    ok = yd > -4                               # where the tanh form has no cancellation in float64
    tanh_form = F.gelu(yd, approximate="tanh")
    assert ((gelu_ref - tanh_form)[ok].abs() <= 1e-12 * (1 + tanh_form[ok].abs())).all()
    close(gl, r(gelu_ref), "gelu")

    h1 = (torch.randn(B, L, D, device="cuda", generator=g) * 2).to(dt)
    h2 = (torch.randn(B, L, D, device="cuda", generator=g) * 2).to(dt)
    skip = torch.randn(B, L, D, device="cuda", generator=g)
    yf, f1, f2 = y.double(), h1.double(), h2.double()
    want = {_lib.M3_ACT_GELU: r(gelu_ref),
            _lib.M3_ACT_FULL_GLU: r(f1 * r(torch.sigmoid(f2))),
            _lib.M3_ACT_HALF_GLU1: r(r(gelu_ref) * r(torch.sigmoid(f2))),
            _lib.M3_ACT_HALF_GLU2: r(yf * r(torch.sigmoid(f2)))}
    for act, v in want.items():
        out = torch.empty_like(skip)
        _lib.check(lib.m3_block_act(y.data_ptr(), h1.data_ptr(), h2.data_ptr(), skip.data_ptr(), out.data_ptr(),
                                    B, L, D, act, io, st), "m3_block_act")
        # out = float32(skip + v): v may differ by its own tolerance, the add by one float32 rounding
        want_out = (skip.double() + v).float().double()
        tol = v.abs() * (2 ** -7 * 1.01 if bf16 else 2e-6) + want_out.abs() * 2 ** -23 + 1e-30
        bad = ((out.double() - want_out).abs() > tol).sum().item()
        assert bad == 0, f"act {act}: {bad} elements outside tolerance"
        # the fused epilogue + LayerNorm: the same sum, bit for bit, then the norm of it
        # (prenorm: sum kept, norm in the compute dtype; postnorm: only the float32 norm)
        ln_want = F.layer_norm(out.double(), (D,), sc.double(), bi.double(), eps=1e-6)
        out2 = torch.empty_like(skip)
        lno = torch.empty(B, L, D, device="cuda", dtype=dt)
        _lib.check(lib.m3_block_act_norm(y.data_ptr(), h1.data_ptr(), h2.data_ptr(), skip.data_ptr(), out2.data_ptr(),
                                         sc.data_ptr(), bi.data_ptr(), lno.data_ptr(), B, L, D, 1e-6, act, io, io,
                                         st), "m3_block_act_norm")
        if bf16:   # the rounding to bf16 before the add leaves one way to evaluate the sum
            assert torch.equal(out2, out), f"act {act}: fused sum differs from m3_block_act"
        else:      # float32: the compiler may fuse skip + x * rcp(..) into one FMA on one path; the
            # difference is the product's rounding, half an ulp of |act| <= |out| + |skip|
            tol = (2 * out.abs() + skip.abs()) * 2 ** -23 + 1e-30
            assert ((out2 - out).abs() <= tol).all(), f"act {act}: fused sum"
        got = lno.double()
        if bf16:   # near-zero normalised values carry the float32 mean's rounding: 1e-6 absolute floor
            bad = ((got - r(ln_want)).abs() > r(ln_want).abs() * 2 ** -7 * 1.01 + 1e-6).sum().item()
            assert bad == 0, f"act {act}: {bad} normalised elements outside tolerance"
        else:
            assert ((got - ln_want).abs().max() / ln_want.abs().max()).item() <= 2e-6
        # in place on the residual (out = skip), as the header allows
        sk2, ln2 = skip.clone(), torch.empty_like(lno)
        _lib.check(lib.m3_block_act_norm(y.data_ptr(), h1.data_ptr(), h2.data_ptr(), sk2.data_ptr(), sk2.data_ptr(),
                                         sc.data_ptr(), bi.data_ptr(), ln2.data_ptr(), B, L, D, 1e-6, act, io, io,
                                         st), "m3_block_act_norm in place")
        assert torch.equal(sk2, out2) and torch.equal(ln2, lno), f"act {act}: in-place act_norm"
        lnf = torch.empty_like(skip)
        _lib.check(lib.m3_block_act_norm(y.data_ptr(), h1.data_ptr(), h2.data_ptr(), skip.data_ptr(), None,
                                         sc.data_ptr(), bi.data_ptr(), lnf.data_ptr(), B, L, D, 1e-6, act, io,
                                         _lib.DTYPE_F32, st), "m3_block_act_norm postnorm")
        assert ((lnf.double() - ln_want).abs().max() / ln_want.abs().max()).item() <= 2e-6

    # the head's log_softmax over rows of width D (in place), against float64
    logits = torch.randn(B, L, D, device="cuda", generator=g) * 4
    want = torch.log_softmax(logits.double(), dim=-1)
    _lib.check(lib.m3_log_softmax(logits.data_ptr(), logits.data_ptr(), B, L, D, st), "m3_log_softmax")
    assert ((logits.double() - want).abs() <= 1e-6 * (1 + want.abs())).all(), "log_softmax"


def test_layer_post_with_a_scale_that_is_not_16_byte_aligned():
    """m3_layer_post's 16-byte path reads the norm scale eight at a time; a scale
    pointer that is only 4-byte aligned takes the element path, with the same result."""
    import torch
    from mamba3_rocm import _lib
    lib = _lib.load()
    B, L, D = 2, 37, 768
    g = torch.Generator(device="cuda")
    g.manual_seed(71)
    y = torch.randn(B, L, D, device="cuda", generator=g).to(torch.bfloat16)
    buf = torch.empty(D + 1, device="cuda")
    buf[1:] = 1.0 + 0.1 * torch.randn(D, device="cuda", generator=g)
    offset = buf[1:]                                    # 4 bytes past a 16-byte boundary
    aligned = offset.clone()
    assert offset.data_ptr() % 16 == 4 and aligned.data_ptr() % 16 == 0
    outs = []
    for scale in (aligned, offset):
        out = torch.empty_like(y)
        stream = torch.cuda.current_stream().cuda_stream
        rc = lib.m3_layer_post(y.data_ptr(), scale.data_ptr(), out.data_ptr(), B, L, D, 1e-6, _lib.DTYPE_BF16,
                               stream)
        assert rc == 0, lib.m3_last_error()
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0].float()).all()
    assert torch.equal(outs[0], outs[1])
