"""Pins of the mixer-layer oracle (oracle/mamba3_layer.py), CPU only.

The layer composes the pinned scan oracle with simple maps; these checks fix
the composition: the shared-B/C path equals the per-head path the reference
also takes (B and C repeated over heads before BCNorm, mamba3.py:236-242 and
265-268), RMSNorm and softplus identities, the decay floor, and linearity of the
output projection.
"""
import numpy as np
import pytest

from oracle import mamba3_layer as ML
from oracle import mamba3_ref as M


def _case(seed=0, B=2, L=70, d_model=32, N=16, headdim=16):
    p = ML.init_params(d_model, seed, d_state=N, headdim=headdim)
    x = np.random.default_rng(seed + 1).standard_normal((B, L, d_model)).astype(np.float32)
    return p, x


def _per_head_path(p, x, N, headdim, chunk):
    """The reference's non-shared preprocessing: B, C and angles repeated over heads
    (mamba3.py:236-238, 265-268), BCNorm per head row, per-head scan."""
    B, L, d_model = x.shape
    nh, hd, R, _ = ML.dims(d_model, N, 2, headdim)
    di = nh * hd
    proj = x.astype(np.float64) @ p["in_proj"].astype(np.float64)
    cut = np.cumsum([di, di, N, N, nh, nh, nh])
    z, xv, Bm, Cm, dd_dt, dd_A, trap, ang = np.split(proj, cut, axis=-1)
    Brep = np.repeat(Bm[:, :, None, :], nh, axis=2)
    Crep = np.repeat(Cm[:, :, None, :], nh, axis=2)
    Bn, Cn = ML.rmsnorm(Brep, p["B_norm"]), ML.rmsnorm(Crep, p["C_norm"])
    A = np.minimum(-ML.softplus(dd_A), -1e-4)
    DT = ML.softplus(dd_dt + p["dt_bias"])
    y = M.mamba3_ssd_chunked_batched(
        Cn, Bn, xv.reshape(B, L, nh, hd), np.transpose(A * DT, (0, 2, 1)), np.transpose(DT, (0, 2, 1)),
        np.transpose(trap, (0, 2, 1)), np.repeat(ang[:, :, None, :], nh, axis=2), p["C_bias"], p["B_bias"],
        p["D"], z.reshape(B, L, nh, hd), chunk_size=chunk).reshape(B, L, di)
    y = y / np.sqrt(np.mean(y * y, axis=-1, keepdims=True) + ML.EPS) * p["out_norm"]
    return y @ p["out_proj"].astype(np.float64)


def test_shared_path_equals_per_head_path():
    p, x = _case()
    a = ML.layer_forward(p, x, d_state=16, headdim=16, chunk_size=16)
    b = _per_head_path(p, x, 16, 16, 16)
    assert np.abs(a - b).max() <= 1e-12 * np.abs(b).max()


def test_rmsnorm_and_softplus_identities():
    x = np.random.default_rng(3).standard_normal((5, 40)) * 7
    y = ML.rmsnorm(x, np.ones(40))
    assert np.allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, atol=1e-6)
    s = np.random.default_rng(4).standard_normal(40)
    assert np.allclose(ML.rmsnorm(x, s), y * s)
    t = np.linspace(-30, 30, 101)
    assert np.allclose(ML.softplus(t) - ML.softplus(-t), t, atol=1e-12)
    assert np.all(np.minimum(-ML.softplus(t), -1e-4) <= -1e-4)


def test_output_projection_is_linear_and_chunk_invariant():
    p, x = _case(seed=5)
    base = ML.layer_forward(p, x, d_state=16, headdim=16, chunk_size=16)
    q = dict(p, out_proj=p["out_proj"] * 2)
    assert np.allclose(ML.layer_forward(q, x, d_state=16, headdim=16, chunk_size=16), 2 * base, rtol=1e-12,
                       atol=1e-12)
    assert np.allclose(ML.layer_forward(p, x, d_state=16, headdim=16, chunk_size=8), base, rtol=1e-9,
                       atol=1e-12)


def test_dims_follow_setup():
    # model geometry: d_model 768, expand 2 -> 24 heads of 64, 32 rope pairs
    nh, hd, R, dproj = ML.dims(768)
    assert (nh, hd, R) == (24, 64, 32)
    assert dproj == 2 * 1536 + 2 * 128 + 3 * 24 + 32


def test_stack_oracle_identities():
    """LayerNorm and gelu identities, and a block whose mixer outputs zero is the
    identity (prenorm) or LayerNorm of its input (postnorm), for every activation."""
    from oracle import mamba3_stack as MS
    x = np.random.default_rng(6).standard_normal((3, 50)) * 4 + 2
    y = MS.layernorm(x, np.ones(50), np.zeros(50))
    assert np.allclose(y.mean(-1), 0, atol=1e-12) and np.allclose(y.std(-1), 1, atol=1e-5)
    t = np.linspace(-6, 6, 61)
    assert np.allclose(MS.gelu(t) - MS.gelu(-t), t, atol=1e-12) and MS.gelu(0.0) == 0.0
    p = MS.init_params(vocab=11, d_model=32, n_layers=1, seed=7, d_state=16, headdim=16)
    lp = p["layers"][0]
    lp["mixer"]["out_proj"] = np.zeros_like(lp["mixer"]["out_proj"])
    ids = np.random.default_rng(8).integers(0, 11, size=(2, 20))
    emb = p["embed"][ids].astype(np.float64)
    for act in MS.ACTIVATIONS:
        if act == "full_glu":       # out1(0) + bias, gated: not zero by construction
            continue
        out = MS.stack_forward(p, ids, activation=act, prenorm=True, d_state=16, headdim=16)
        assert np.allclose(out, emb, atol=1e-12), act
        out = MS.stack_forward(p, ids, activation=act, prenorm=False, d_state=16, headdim=16)
        assert np.allclose(out, MS.layernorm(emb, lp["ln_scale"], lp["ln_bias"]), atol=1e-12), act


def test_lm_head_is_normalised_and_shift_invariant():
    """Each token's log-probabilities sum to one in probability, and a constant added
    to every decoder bias leaves them unchanged."""
    from oracle import mamba3_stack as MS
    p = MS.init_params(vocab=13, d_model=32, n_layers=1, seed=9, d_state=16, headdim=16)
    ids = np.random.default_rng(10).integers(0, 13, size=(2, 24))
    lp = MS.lm_forward(p, ids, d_state=16, headdim=16)
    assert lp.shape == (2, 24, 13)
    assert np.allclose(np.exp(lp).sum(-1), 1.0, atol=1e-12)
    q = dict(p, decoder_b=p["decoder_b"] + 3.5)
    assert np.allclose(MS.lm_forward(q, ids, d_state=16, headdim=16), lp, atol=1e-12)
    feats = MS.stack_forward(p, ids, d_state=16, headdim=16)
    z = feats @ p["decoder_w"].astype(np.float64) + p["decoder_b"]
    assert np.allclose(np.argmax(lp, -1), np.argmax(z, -1))


def test_stack_oracle_glu_variants_closed_forms():
    """The GLU activations of layers.py:126-141 with m the mixer output and g = gelu(m):
    full_glu = out1(g) sigmoid(out2(g)), half_glu1 = g sigmoid(out2(g)),
    half_glu2 = m sigmoid(out2(g)).  Two special cases fix the wiring:
    (1) out2's kernel zero and bias b: the gate is the constant sigmoid(b), so the
        gated tensor shows (g, m, or out1(g));
    (2) out2 = alpha I without bias and out1 = I: the gate is sigmoid(alpha g), so a
        gate fed m instead of g, or out1 and out2 swapped, fails."""
    from oracle import mamba3_stack as MS
    D = 32
    p = MS.init_params(vocab=11, d_model=D, n_layers=1, seed=12, d_state=16, headdim=16)
    lp = p["layers"][0]
    ids = np.random.default_rng(13).integers(0, 11, size=(2, 20))
    emb = p["embed"][ids].astype(np.float64)
    m = ML.layer_forward(lp["mixer"], MS.layernorm(emb, lp["ln_scale"], lp["ln_bias"]), d_state=16, headdim=16)
    g = MS.gelu(m)
    assert np.abs(m).max() > 0.1 and np.abs(g - m).max() > 0.1, "the mixer output must be non-trivial"

    def block(act):   # prenorm: x + act(mixer(LN(x)))
        return MS.stack_forward(p, ids, activation=act, prenorm=True, d_state=16, headdim=16) - emb

    b = np.random.default_rng(14).standard_normal(D)
    lp["out2_w"], lp["out2_b"] = np.zeros((D, D), np.float32), b.astype(np.float32)
    s = MS.sigmoid(b.astype(np.float32).astype(np.float64))
    out1 = g @ lp["out1_w"].astype(np.float64) + lp["out1_b"]
    assert np.allclose(block("half_glu1"), g * s, atol=1e-10)
    assert np.allclose(block("half_glu2"), m * s, atol=1e-10)
    assert np.allclose(block("full_glu"), out1 * s, atol=1e-10)

    alpha = 3.0
    lp["out2_w"], lp["out2_b"] = (alpha * np.eye(D)).astype(np.float32), np.zeros(D, np.float32)
    lp["out1_w"], lp["out1_b"] = np.eye(D, dtype=np.float32), np.zeros(D, np.float32)
    gate = MS.sigmoid(alpha * g)
    assert np.allclose(block("half_glu1"), g * gate, atol=1e-10)
    assert np.allclose(block("half_glu2"), m * gate, atol=1e-10)
    assert np.allclose(block("full_glu"), g * gate, atol=1e-10)
    assert not np.allclose(block("half_glu2"), m * MS.sigmoid(alpha * m), atol=1e-3)


# ---------------------------------------------------------------- wiring pins
# The split order of in_proj's output and the decay are fixed here by special
# parameters whose layer output has a form computed without the oracle's own split
# (the column offsets below are written out from mamba3.py:212-219's order
# [z, x, B, C, dd_dt, dd_A, trap, angles]), so that a swapped block fails.
WIRE = dict(d_model=32, N=16, headdim=16)


def _offsets(d_model, N, headdim):
    nh, hd, R, dproj = ML.dims(d_model, N, 2, headdim)
    di = nh * hd
    o = {"z": 0, "x": di, "B": 2 * di, "C": 2 * di + N, "dd_dt": 2 * di + 2 * N}
    o["dd_A"] = o["dd_dt"] + nh
    o["trap"] = o["dd_A"] + nh
    o["ang"] = o["trap"] + nh
    assert o["ang"] + R == dproj
    return nh, hd, R, di, o


def _out_norm_proj(p, y):
    """_post_norm_and_project (mamba3.py:281-325) on float64 y (B, L, d_inner)."""
    yn = y / np.sqrt(np.mean(y * y, axis=-1, keepdims=True) + ML.EPS)
    return (yn * p["out_norm"]) @ p["out_proj"].astype(np.float64)


def _skip_only_case(seed=20):
    """B, C and angle columns of in_proj zero, B and C biases zero: the normalised B
    and C rows are zero, so the scan is its skip term alone, y = D x silu(z)."""
    d_model, N, headdim = WIRE["d_model"], WIRE["N"], WIRE["headdim"]
    p = ML.init_params(d_model, seed, d_state=N, headdim=headdim)
    nh, hd, R, di, o = _offsets(d_model, N, headdim)
    W = p["in_proj"].copy()
    W[:, o["B"]:o["dd_dt"]] = 0.0
    W[:, o["ang"]:] = 0.0
    p.update(in_proj=W, B_bias=np.zeros_like(p["B_bias"]), C_bias=np.zeros_like(p["C_bias"]))
    x = np.random.default_rng(seed + 1).standard_normal((2, 40, d_model)).astype(np.float32)
    proj = x.astype(np.float64) @ W.astype(np.float64)
    B_, L = x.shape[:2]
    xv = proj[..., o["x"]:o["x"] + di].reshape(B_, L, nh, hd)
    z = proj[..., o["z"]:o["z"] + di].reshape(B_, L, nh, hd)
    y = (p["D"][:, None] * xv * z / (1 + np.exp(-z))).reshape(B_, L, di)
    return p, x, _out_norm_proj(p, y)


def _constant_feature_case(seed=21):
    """The input's last feature is 1 and the dd_dt, dd_A, trap and angle columns of
    in_proj are zero except in that feature's row: every token of a head sees the
    same chosen dd_dt, dd_A, trap and angle rate.  The expected output is the
    brute-force quadratic form (oracle/pins.py) on inputs cut from the projection at
    the reference's offsets, with A = -softplus(dd_A) and DT = softplus(dd_dt +
    dt_bias) formed here."""
    from oracle import pins
    d_model, N, headdim = WIRE["d_model"], WIRE["N"], WIRE["headdim"]
    p = ML.init_params(d_model, seed, d_state=N, headdim=headdim)
    nh, hd, R, di, o = _offsets(d_model, N, headdim)
    rng = np.random.default_rng(seed + 1)
    consts = {"dd_dt": rng.uniform(-1.5, 0.5, nh), "dd_A": rng.uniform(-0.5, 2.0, nh),
              "trap": rng.uniform(-1.5, 1.5, nh), "ang": rng.uniform(-2.0, 2.0, R)}
    consts = {k: c.astype(np.float32).astype(np.float64) for k, c in consts.items()}   # in_proj is float32
    W = p["in_proj"].copy()
    for k, c in consts.items():
        W[:, o[k]:o[k] + len(c)] = 0.0
        W[-1, o[k]:o[k] + len(c)] = c
    p["in_proj"] = W.astype(np.float32)
    L = 24
    x = rng.standard_normal((1, L, d_model)).astype(np.float32)
    x[..., -1] = 1.0
    proj = (x.astype(np.float64) @ p["in_proj"].astype(np.float64))[0]
    A = -np.log1p(np.exp(consts["dd_A"]))
    DT = np.log1p(np.exp(consts["dd_dt"] + p["dt_bias"].astype(np.float64)))
    assert np.all(A < -1e-4)                                   # above the floor
    cols = lambda k, w: proj[:, o[k]:o[k] + w]                  # noqa: E731
    Cn, Bn = ML.rmsnorm(cols("C", N), p["C_norm"]), ML.rmsnorm(cols("B", N), p["B_norm"])
    rep = lambda a: np.repeat(a[:, None, :], nh, axis=1)        # noqa: E731
    y = pins.quadratic_form(
        rep(Cn), rep(Bn), cols("x", di).reshape(L, nh, hd),
        np.repeat((A * DT)[:, None], L, axis=1), np.repeat(DT[:, None], L, axis=1),
        np.repeat(consts["trap"][:, None], L, axis=1), np.broadcast_to(consts["ang"], (L, nh, R)),
        p["C_bias"], p["B_bias"], p["D"], cols("z", di).reshape(L, nh, hd))
    return p, x, _out_norm_proj(p, y.reshape(1, L, di))


def test_layer_oracle_skip_term_fixes_z_and_x():
    p, x, want = _skip_only_case()
    got = ML.layer_forward(p, x, d_state=WIRE["N"], headdim=WIRE["headdim"], chunk_size=16)
    assert np.abs(got - want).max() <= 1e-10 * np.abs(want).max()


def test_layer_oracle_wiring_matches_quadratic_form():
    p, x, want = _constant_feature_case()
    got = ML.layer_forward(p, x, d_state=WIRE["N"], headdim=WIRE["headdim"], chunk_size=8)
    assert np.abs(got - want).max() <= 1e-9 * np.abs(want).max()


def _plant_wiring(monkeypatch, which):
    split = ML.split_proj

    def swapped(proj, di, N, nh):
        z, xv, Bm, Cm, dd_dt, dd_A, trap, ang = split(proj, di, N, nh)
        if which == "z_x":
            z, xv = xv, z
        elif which == "B_C":
            Bm, Cm = Cm, Bm
        elif which == "dd_dt_dd_A":
            dd_dt, dd_A = dd_A, dd_dt
        elif which == "dd_A_trap":
            dd_A, trap = trap, dd_A
        return z, xv, Bm, Cm, dd_dt, dd_A, trap, ang
    monkeypatch.setattr(ML, "split_proj", swapped)


@pytest.mark.parametrize("which", ["z_x", "B_C", "dd_dt_dd_A", "dd_A_trap"])
def test_planted_wiring_swaps_fail_the_pins(monkeypatch, which):
    cases = [_constant_feature_case()] + ([_skip_only_case()] if which == "z_x" else [])
    _plant_wiring(monkeypatch, which)
    for p, x, want in cases:
        got = ML.layer_forward(p, x, d_state=WIRE["N"], headdim=WIRE["headdim"], chunk_size=8)
        assert np.abs(got - want).max() > 1e-3 * np.abs(want).max(), which


def test_planted_decay_mistake_fails_the_pin(monkeypatch):
    """A decay that forgets the dt bias (DT = softplus(dd_dt)) fails the wiring pin."""
    monkeypatch.setattr(ML, "decay", lambda dd_dt, dd_A, dt_bias, A_floor:
                        (np.minimum(-ML.softplus(dd_A), -A_floor), ML.softplus(dd_dt)))
    p, x, want = _constant_feature_case()
    got = ML.layer_forward(p, x, d_state=WIRE["N"], headdim=WIRE["headdim"], chunk_size=8)
    assert np.abs(got - want).max() > 1e-3 * np.abs(want).max()
