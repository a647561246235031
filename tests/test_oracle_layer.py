"""Pins of the mixer-layer oracle (oracle/mamba3_layer.py), CPU only.

The layer composes the pinned scan oracle with simple maps; these checks fix
the composition: the shared-B/C path equals the per-head path the reference
also takes (B and C repeated over heads before BCNorm, mamba3.py:236-242 and
265-268), RMSNorm and softplus identities, the decay floor, and linearity of the
output projection.
"""
import numpy as np

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
