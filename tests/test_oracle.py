"""Pins of the CPU oracle (no GPU).

The reference commits no golden vectors for this path and its JAX code is
not importable here, so the restatement in oracle/mamba3_ref.py is pinned by
what the mathematics fixes:
  * the brute-force quadratic (attention) form, written independently
    (complex-number rotation, scalar accumulation) in oracle/pins.py;
  * the token-by-token decode recurrence: chunked == recurrent is the
    reference's own contract (tests/integration/test_backbone_contracts.py:81-111);
  * chunk-size invariance (the dense and blocked state passes agree,
    tests/unit/test_mamba3_pallas_ssd.py:223-241);
  * a textbook special case: no decay, no rotation, sigmoid(trap) = 1 and
    zero biases reduce the scan to causal linear attention
    y_t = sum_{s<=t} dt_s (q_t . k_s) v_s;
  * closed forms and invariants of each piece (rope, angle cumsum, trapezoid);
  * planted mistakes (a dropped term, a sign flip, an inclusive mask, a
    shifted trapezoid weight) that each of these checks must catch.
"""
import numpy as np
import pytest

from oracle import inputs as I
from oracle import mamba3_ref as M
from oracle import pins

# (L, H, N, R, P, CS): the reference's unit-test shapes (test_mamba3_pallas_ssd.py:32-36)
# plus tiny and odd shapes.
SHAPES = [(70, 2, 64, 16, 16, 16), (128, 3, 64, 32, 16, 32), (200, 2, 128, 32, 32, 64),
          (13, 2, 8, 2, 4, 4), (37, 1, 16, 0, 8, 8), (19, 2, 12, 3, 6, 5)]


def _args(L, H, N, R, P, seed, bf16=False):
    d = I.scan_inputs(1, L, H, N, P, R, seed=seed, bf16=bf16)
    return (d["Q"][0], d["K"][0], d["V"][0], d["ADT"][0], d["DT"][0], d["Trap"][0],
            d["Angles"][0], d["Q_bias"], d["K_bias"], d["D"], d["Z"][0])


def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


def _recurrent(args):
    Q, K, V, ADT, DT, Trap, Ang, qb, kb, D, Z = args
    H, N, P, R = Q.shape[1], Q.shape[2], V.shape[2], Ang.shape[2]
    carry = (np.zeros((H, R)), np.zeros((H, P, N)), np.zeros((H, N)), np.zeros((H, P)))
    _, y = M.rnn_scan(carry, pins.seq_inputs_from_scan_args(Q, K, V, ADT, DT, Trap, Ang, Z),
                      kb, qb, D)
    return y


@pytest.mark.parametrize("L,H,N,R,P,CS", SHAPES)
@pytest.mark.parametrize("seed", [0, 1])
def test_chunked_matches_quadratic_form(L, H, N, R, P, CS, seed):
    a = _args(L, H, N, R, P, seed)
    y = M.mamba3_ssd_chunked(*a, chunk_size=CS)
    q = pins.quadratic_form(*a)
    assert y.shape == (L, H, P)
    assert _rel(y, q) < 1e-12


@pytest.mark.parametrize("L,H,N,R,P,CS", SHAPES[:4])
def test_recurrence_matches_quadratic_form(L, H, N, R, P, CS):
    a = _args(L, H, N, R, P, seed=2)
    assert _rel(_recurrent(a), pins.quadratic_form(*a)) < 1e-12


def test_chunk_size_invariance():
    a = _args(150, 2, 32, 8, 16, seed=3)
    ys = [M.mamba3_ssd_chunked(*a, chunk_size=cs) for cs in (1, 4, 7, 16, 64, 150, 256)]
    for y in ys[1:]:
        assert _rel(y, ys[0]) < 1e-12


def test_reduces_to_causal_linear_attention():
    """A = 0, R = 0, sigmoid(trap) = 1, zero biases, D = 0, no gate."""
    rng = np.random.default_rng(4)
    L, H, N, P = 90, 2, 16, 8
    Q = rng.standard_normal((L, H, N))
    K = rng.standard_normal((L, H, N))
    V = rng.standard_normal((L, H, P))
    DT = rng.uniform(0.1, 1.0, (H, L))
    ADT = np.zeros((H, L))
    Trap = np.full((H, L), 60.0)          # sigmoid == 1.0 exactly in float64
    ang = np.zeros((L, H, 0))
    zb = np.zeros((H, N))
    y = M.mamba3_ssd_chunked(Q, K, V, ADT, DT, Trap, ang, zb, zb, None, None, chunk_size=16)
    # textbook: H_t = sum_{s<=t} dt_s k_s (x) v_s ; y_t = q_t . H_t
    kv = np.einsum("lhn,lhp->lhnp", K * DT.T[..., None], V)
    Hs = np.cumsum(kv, axis=0)
    ref = np.einsum("lhn,lhnp->lhp", Q, Hs)
    assert _rel(y, ref) < 1e-12


def test_decay_only_closed_form():
    """N = 2, R = 0, sigmoid(trap) = 1, single head: y_t = sum_{s<=t} e^{A_t - A_s} dt_s (q_t.k_s) v_s."""
    rng = np.random.default_rng(5)
    L = 40
    Q = rng.standard_normal((L, 1, 2))
    K = rng.standard_normal((L, 1, 2))
    V = rng.standard_normal((L, 1, 1))
    DT = rng.uniform(0.1, 0.5, (1, L))
    ADT = -rng.uniform(0.0, 0.7, (1, L))
    Trap = np.full((1, L), 60.0)
    zb = np.zeros((1, 2))
    y = M.mamba3_ssd_chunked(Q, K, V, ADT, DT, Trap, np.zeros((L, 1, 0)), zb, zb, None, None,
                             chunk_size=8)
    A = np.cumsum(ADT[0])
    ref = np.zeros(L)
    for t in range(L):
        for s in range(t + 1):
            ref[t] += np.exp(A[t] - A[s]) * DT[0, s] * (Q[t, 0] @ K[s, 0]) * V[s, 0, 0]
    assert _rel(y[:, 0, 0], ref) < 1e-12


def test_rope_properties():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((5, 3, 16))
    k = rng.standard_normal((5, 3, 16))
    th = rng.uniform(0, 2 * np.pi, (5, 3, 5))
    xr = M.apply_rope(x, np.cos(th), np.sin(th))
    kr = M.apply_rope(k, np.cos(th), np.sin(th))
    assert np.allclose(np.linalg.norm(xr, axis=-1), np.linalg.norm(x, axis=-1))
    assert np.allclose(np.sum(xr * kr, -1), np.sum(x * k, -1))     # equal angles keep q.k
    assert np.array_equal(xr[..., 10:], x[..., 10:])                 # pairs >= R pass through
    for idx in np.ndindex(5, 3):                                      # complex rotation
        assert np.allclose(xr[idx], pins._rot(x[idx], th[idx]))


def test_angle_cumsum_closed_form():
    rng = np.random.default_rng(7)
    ang = rng.uniform(-np.pi, np.pi, (300, 2, 4))
    dt = rng.uniform(0.0, 0.5, (2, 300))
    th = M.angle_dt_cumsum(ang, dt)
    assert (th >= 0).all() and (th < 2 * np.pi).all()
    raw = np.cumsum(np.tanh(ang) * np.pi * dt.T[..., None], axis=0)
    assert np.allclose(np.mod(raw, 2 * np.pi), th, atol=1e-9)


def test_trapezoid_closed_form():
    rng = np.random.default_rng(8)
    DT = rng.uniform(0, 1, (2, 9))
    Trap = rng.standard_normal((2, 9))
    g, s = M.trapezoid_gamma_scale(DT, Trap)
    sig = 1 / (1 + np.exp(-Trap))
    assert np.allclose(g, DT * sig)
    exp_s = DT * sig
    exp_s[:, :-1] += DT[:, 1:] * (1 - sig[:, 1:])
    assert np.allclose(s, exp_s)


def test_float32_mode_tracks_float64():
    a = _args(200, 2, 128, 32, 32, seed=9, bf16=True)
    y64 = M.mamba3_ssd_chunked(*a, chunk_size=64)
    y32 = M.mamba3_ssd_chunked(*a, chunk_size=64, dtype=np.float32)
    assert y32.dtype == np.float32
    assert _rel(y32, y64) < 1e-5


def test_rnn_step_modes():
    d = I.decode_inputs(3, 2, 16, 8, 4, 1, seed=10, bf16=False)
    carry = tuple(d[k] for k in ("theta", "h", "k_prev", "v_prev"))
    tin = tuple(d[k][0] for k in ("x", "z", "Bt", "Ct", "adt", "dt", "trap", "ang"))
    c0, y0 = M.rnn_step(carry, tin, d["B_bias"], d["C_bias"], d["D"])
    c1, y1 = M.rnn_step(carry, tin, d["B_bias"], d["C_bias"], d["D"], diag_mode="legacy_double")
    # legacy_double adds gamma (C_rot . B_rot) x_t once more, gated by silu(z) (mamba3.py:549-559)
    gamma = d["dt"][0] * d["trap"][0]
    qk = np.sum(c0[2] * M.apply_rope(d["Ct"][0] + d["C_bias"], np.cos(c0[0]), np.sin(c0[0])), -1)
    z = d["z"][0]
    extra = (qk * gamma)[..., None] * d["x"][0] * z / (1 + np.exp(-z))
    assert np.allclose(y1 - y0, extra)
    c2, y2 = M.rnn_step(carry, tin, d["B_bias"], d["C_bias"], d["D"], angle_mode="legacy_unbounded")
    assert np.allclose(y2, y0)                        # same rotation, unwrapped state
    assert np.allclose(np.mod(c2[0], 2 * np.pi), c0[0])
    with pytest.raises(ValueError):
        M.rnn_step(carry, tin, d["B_bias"], d["C_bias"], d["D"], angle_mode="bogus")


# ------------------------------------------------------------ planted mistakes
def _plant(monkeypatch, which):
    if which == "no_shift":      # trapezoid scale without the next token's term
        def tg(DT, Trap):
            sig = 1 / (1 + np.exp(-Trap))
            g = DT * sig
            return g, g
        monkeypatch.setattr(M, "trapezoid_gamma_scale", tg)
    elif which == "rope_sign":   # rotation in the wrong direction
        orig = M.apply_rope
        monkeypatch.setattr(M, "apply_rope", lambda x, c, s: orig(x, c, -s))
    elif which == "shift_wrong_side":  # shifted weight taken from the previous token
        def tg(DT, Trap):
            sig = 1 / (1 + np.exp(-Trap))
            g = DT * sig
            sh = np.pad((DT * (1 - sig))[:, :-1], ((0, 0), (1, 0)))
            return g, g + sh
        monkeypatch.setattr(M, "trapezoid_gamma_scale", tg)
    elif which == "no_decay_state":  # states passed without the chunk decay
        orig = M.phases_4_5_6
        monkeypatch.setattr(M, "phases_4_5_6", lambda Qc, Kc, Vc, Ac, Acum: orig(Qc, Kc, Vc, Ac, Acum * 0))


@pytest.mark.parametrize("which", ["no_shift", "rope_sign", "shift_wrong_side", "no_decay_state"])
def test_planted_mistakes_fail_the_pins(monkeypatch, which):
    a = _args(70, 2, 32, 8, 16, seed=11)
    q = pins.quadratic_form(*a)
    _plant(monkeypatch, which)
    y = M.mamba3_ssd_chunked(*a, chunk_size=16)
    assert _rel(y, q) > 1e-3, which


def test_planted_recurrence_mistake_fails():
    """Dropping the (1 - trap) previous-token term in rnn_step breaks chunked == recurrent."""
    a = _args(40, 2, 16, 4, 8, seed=12)
    q = pins.quadratic_form(*a)
    Q, K, V, ADT, DT, Trap, Ang, qb, kb, D, Z = a
    seq = pins.seq_inputs_from_scan_args(Q, K, V, ADT, DT, Trap, Ang, Z)
    H, N, P, R = 2, 16, 8, 4
    carry = (np.zeros((H, R)), np.zeros((H, P, N)), np.zeros((H, N)), np.zeros((H, P)))
    ys = []
    for t in range(40):
        x_t, z_t, B_t, C_t, adt, dt, trap, ang = (s[t] for s in seq)
        carry = (carry[0], carry[1], carry[2] * 0, carry[3])   # planted: forget k_prev
        carry, y = M.rnn_step(carry, (x_t, z_t, B_t, C_t, adt, dt, trap, ang), kb, qb, D)
        ys.append(y)
    assert _rel(np.stack(ys), q) > 1e-3
