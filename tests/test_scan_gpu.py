"""Prefill scan on the GPU vs the CPU oracle (parity gate).

Tolerances: fp32 runs max-rel-err <= 1e-4 against
the float64 oracle; bf16 runs (fp32 accumulate) <= 2e-2 against the oracle on
the same bf16-rounded inputs.  The error metric is the reference's _rel
(test_mamba3_pallas_ssd.py:79-82).  Shapes cover the reference's own test
shapes (test_mamba3_pallas_ssd.py:32-36, ragged L), the GPU test shape
(test_mamba3_pallas_gpu.py:27), GQA, optional D/Z, L < chunk and the headline
configuration, the latter through per-(batch, head) subsets and chunk-size
invariance.
"""
import numpy as np
import pytest

from _util import I, M, hip_scan, oracle_scan, rel, to_dev

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2


def _torch():
    import torch
    return torch


def _run(B, L, H, N, P, R, CS, bf16, seed, Hqk=None, no_d=False, no_z=False):
    torch = _torch()
    d = I.scan_inputs(B, L, H, N, P, R, seed=seed, Hqk=Hqk, bf16=bf16)
    t = to_dev(d, torch.bfloat16 if bf16 else torch.float32)
    got = hip_scan(t, CS, no_d=no_d, no_z=no_z)
    torch.cuda.synchronize()
    ref = oracle_scan(d, CS, no_d=no_d, no_z=no_z)
    out = got.float().cpu().numpy()
    assert got.dtype == (torch.bfloat16 if bf16 else torch.float32)
    assert out.shape == ref.shape == (B, L, H, P)
    assert np.isfinite(out).all()
    return rel(out, ref)


# (B, L, H, N, P, R, CS)
F32_SHAPES = [
    (2, 1024, 8, 64, 64, 16, 64),     # benchmark config 1
    (1, 70, 2, 64, 16, 16, 16),       # reference unit-test shapes (generic kernel for P=16)
    (1, 128, 3, 64, 16, 32, 32),
    (1, 200, 2, 128, 32, 32, 64),
    (1, 1024, 4, 128, 64, 32, 64),    # reference GPU test shape (fp32, N=128): the float32 chunked kernel
    (1, 333, 2, 128, 64, 64, 64),     # fp32 model geometry, rope on every state pair
    (2, 97, 4, 128, 64, 32, 32),      # fp32 model geometry, ragged L, chunk 32
    (1, 300, 2, 128, 64, 32, 128),    # fp32 model geometry, chunk 128: 32-token sub-chunks
    (2, 333, 4, 64, 32, 16, 32),
    (1, 97, 2, 32, 64, 8, 64),
    (1, 300, 2, 64, 64, 16, 128),     # chunk 128: 64-token sub-chunks
]


@pytest.mark.parametrize("B,L,H,N,P,R,CS", F32_SHAPES)
def test_f32_matches_oracle(B, L, H, N, P, R, CS):
    err = _run(B, L, H, N, P, R, CS, bf16=False, seed=1)
    print(f"f32 {(B, L, H, N, P, R, CS)} rel={err:.3e}")
    assert err <= F32_TOL


BF16_SHAPES = [
    (2, 1024, 4, 128, 64, 32, 64),    # headline geometry, fewer heads
    (1, 1061, 3, 128, 64, 32, 64),    # ragged L
    (1, 200, 2, 128, 32, 32, 64),
    (2, 512, 2, 64, 64, 16, 64),
    (1, 300, 2, 128, 64, 32, 32),     # chunk 32
    (1, 257, 2, 64, 32, 16, 32),
    (1, 160, 2, 128, 128, 32, 64),    # P = 128
    (1, 130, 2, 32, 32, 8, 64),
    (1, 77, 2, 128, 64, 64, 64),      # rope on every state pair (R = N/2)
    (1, 77, 2, 128, 64, 0, 64),       # no rope
    (1, 700, 2, 128, 64, 32, 128),    # chunk 128 (config 3's): 64-token sub-chunks
]


@pytest.mark.parametrize("B,L,H,N,P,R,CS", BF16_SHAPES)
def test_bf16_matches_oracle(B, L, H, N, P, R, CS):
    err = _run(B, L, H, N, P, R, CS, bf16=True, seed=2)
    print(f"bf16 {(B, L, H, N, P, R, CS)} rel={err:.3e}")
    assert err <= BF16_TOL


@pytest.mark.parametrize("bf16", [False, True])
def test_short_sequences(bf16):
    for L in (1, 2, 5, 63, 64, 65):
        err = _run(1, L, 2, 64, 64, 16, 64, bf16=bf16, seed=3 + L)
        assert err <= (BF16_TOL if bf16 else F32_TOL), (L, err)


@pytest.mark.parametrize("bf16", [False, True])
def test_gqa_heads(bf16):
    err = _run(2, 300, 4, 64, 64, 16, 64, bf16=bf16, seed=4, Hqk=2)
    assert err <= (BF16_TOL if bf16 else F32_TOL)
    err = _run(1, 300, 4, 64, 64, 16, 64, bf16=bf16, seed=5, Hqk=1)
    assert err <= (BF16_TOL if bf16 else F32_TOL)
    err = _run(1, 200, 4, 128, 64, 32, 64, bf16=bf16, seed=10, Hqk=2)     # the model's geometry
    assert err <= (BF16_TOL if bf16 else F32_TOL)


@pytest.mark.parametrize("bf16", [False, True])
def test_optional_d_and_z(bf16):
    tol = BF16_TOL if bf16 else F32_TOL
    assert _run(1, 150, 2, 64, 64, 16, 64, bf16=bf16, seed=6, no_d=True) <= tol
    assert _run(1, 150, 2, 64, 64, 16, 64, bf16=bf16, seed=7, no_z=True) <= tol
    assert _run(1, 150, 2, 64, 64, 16, 64, bf16=bf16, seed=8, no_d=True, no_z=True) <= tol


def test_unbatched_call_matches_batched():
    torch = _torch()
    from mamba3_rocm import mamba3_siso_hip
    d = I.scan_inputs(1, 200, 2, 128, 64, 32, seed=9, bf16=True)
    t = to_dev(d, torch.bfloat16)
    batched = hip_scan(t, 64)
    un = mamba3_siso_hip(t["Q"][0], t["K"][0], t["V"][0], t["ADT"][0], t["DT"][0], t["Trap"][0],
                         t["Q_bias"], t["K_bias"], t["Angles"][0], t["D"], t["Z"][0], 64)
    assert un.shape == (200, 2, 64)
    assert torch.equal(un, batched[0])


def test_headline_config_subset_and_chunk_invariance():
    """Config 2 (B=8, L=4096, H=32, P=64, N=128, R=32, CS=64, bf16 I/O) at full
    size: four (batch, head) pairs against the float64 oracle, and the whole
    output against the chunk-32 tiling of the same kernel family."""
    torch = _torch()
    B, L, H, N, P, R = 8, 4096, 32, 128, 64, 32
    d = I.scan_inputs(B, L, H, N, P, R, seed=2, bf16=True)
    t = to_dev(d, torch.bfloat16)
    y64 = hip_scan(t, 64)
    y32 = hip_scan(t, 32)
    torch.cuda.synchronize()
    a64 = y64.float().cpu().numpy()
    assert np.isfinite(a64).all()
    assert rel(a64, y32.float().cpu().numpy()) <= BF16_TOL
    for b, h in ((0, 0), (3, 17), (7, 31), (5, 8)):
        sub = {k: (v[b:b + 1] if v.ndim >= 3 or k in ("ADT", "DT", "Trap") else v) for k, v in d.items()}
        ref = M.mamba3_ssd_chunked_batched(
            sub["Q"], sub["K"], sub["V"], sub["ADT"], sub["DT"], sub["Trap"], sub["Angles"],
            d["Q_bias"], d["K_bias"], d["D"], sub["Z"], chunk_size=64, heads=[h])
        err = rel(a64[b:b + 1, :, h:h + 1], ref)
        print(f"config2 b={b} h={h} rel={err:.3e}")
        assert err <= BF16_TOL


@pytest.mark.parametrize("bf16,N,P,R,impl", [(False, 64, 64, 16, 1), (False, 128, 64, 32, 1),
                                              (True, 128, 64, 32, 1), (False, 128, 64, 0, 2),
                                              (True, 48, 16, 12, 2)])
def test_repeat_calls_bitwise_identical(bf16, N, P, R, impl):
    """The kernels use no atomics and no cross-workgroup communication, so repeated
    calls must give bitwise-identical outputs; a race between waves (for example
    a read of per-chunk constants before the wave that writes them) shows up here.
    The last two cases take the generic kernel (impl 2), whose per-row dot products
    are summed in a fixed order."""
    torch = _torch()
    from mamba3_rocm import _lib
    assert _lib.load().m3_chunk_scan_impl(int(bf16), N, P, R, 64) == impl
    B, L, H = ((2, 2048, 16) if bf16 else (2, 1024, 8)) if impl == 1 else (2, 300, 4)
    d = I.scan_inputs(B, L, H, N, P, R, seed=11, bf16=bf16)
    t = to_dev(d, torch.bfloat16 if bf16 else torch.float32)
    first = hip_scan(t, 64)
    for _ in range(4):
        assert torch.equal(hip_scan(t, 64), first)


@pytest.mark.parametrize("bf16", [False, True])
def test_carry_split_equals_full(bf16):
    """Prefill [0, L1) with the carry out, then [L1, L) with it as the carry in,
    equals one prefill over [0, L) -- pins initial/final carry semantics."""
    torch = _torch()
    from mamba3_rocm import mamba3_siso_hip_carry
    B, L, H, N, P, R = 2, 400, 2, 64, 64, 16
    L1 = 137
    d = I.scan_inputs(B, L, H, N, P, R, seed=10, bf16=bf16)
    t = to_dev(d, torch.bfloat16 if bf16 else torch.float32)

    def part(lo, hi, carry):
        s = {k: (v[:, lo:hi] if k in ("Q", "K", "V", "Z", "Angles") else
                 v[:, :, lo:hi] if k in ("ADT", "DT", "Trap") else v) for k, v in t.items()}
        return mamba3_siso_hip_carry(s["Q"], s["K"], s["V"], s["ADT"], s["DT"], s["Trap"],
                                     s["Q_bias"], s["K_bias"], s["Angles"], s["D"], s["Z"], 64,
                                     initial_carry=carry)

    full, fin_full = part(0, L, None)
    y1, c1 = part(0, L1, None)
    y2, c2 = part(L1, L, c1)
    torch.cuda.synchronize()
    tol = BF16_TOL if bf16 else F32_TOL
    ref = oracle_scan(d, 64)
    assert rel(full.float().cpu().numpy(), ref) <= tol
    joined = torch.cat([y1, y2], dim=1).float().cpu().numpy()
    assert rel(joined, ref) <= tol
    th_a, th_b = c2[0].cpu().numpy(), fin_full[0].cpu().numpy()
    assert rel(np.cos(th_a), np.cos(th_b)) <= 1e-4 and rel(np.sin(th_a), np.sin(th_b)) <= 1e-4
    for a, b in zip(c2[1:], fin_full[1:]):
        assert rel(a.cpu().numpy(), b.cpu().numpy()) <= (1e-2 if bf16 else 1e-4)


# (B, L, H, Hqk, R, CS): shapes whose few (batch, head) pairs split the sequence
SPLIT_SHAPES = [
    (1, 1061, 3, 3, 32, 64),     # ragged last segment
    (2, 700, 2, 1, 64, 128),     # GQA (one Q/K head), full-width rope, chunk 128
    (1, 600, 2, 2, 0, 64),       # no rope
    (1, 640, 2, 2, 32, 32),      # chunk 32: the full pass runs other chunks than the state pass
]


@pytest.mark.parametrize("B,L,H,Hqk,R,CS", SPLIT_SHAPES)
def test_sequence_split_matches_oracle_and_single_pass(B, L, H, Hqk, R, CS):
    """bf16 launches with B*H far below the CU count split each sequence into
    segments (state-only pass, carry combine, full pass); the result matches the
    oracle and the one-pass kernel up to rounding."""
    torch = _torch()
    from mamba3_rocm import _lib
    N, P = 128, 64
    assert _lib.load().m3_chunk_scan_ws_bytes(B, L, H, N, P, R, CS, _lib.DTYPE_BF16) > 0
    d = I.scan_inputs(B, L, H, N, P, R, seed=21, Hqk=Hqk, bf16=True)
    t = to_dev(d, torch.bfloat16)
    split = hip_scan(t, CS).float().cpu().numpy()
    single = hip_scan(t, CS, seq_split=False).float().cpu().numpy()
    ref = oracle_scan(d, CS)
    print(f"split {(B, L, H, Hqk, R, CS)} rel={rel(split, ref):.3e} vs single {rel(split, single):.3e}")
    assert np.isfinite(split).all()
    assert rel(split, ref) <= BF16_TOL
    assert rel(split, single) <= BF16_TOL


@pytest.mark.parametrize("B,L,H,Hqk,R,CS", [
    (1, 1061, 3, 3, 32, 64),     # ragged last segment
    (2, 700, 2, 1, 64, 128),     # GQA, full-width rope, chunk 128
    (1, 640, 2, 2, 32, 32),
])
def test_sequence_split_float32(B, L, H, Hqk, R, CS):
    """float32 I/O (what the model's mamba3_siso_triton call receives) splits the
    sequence too: the float32 kernel's state-only pass, the combine and its full
    pass match the oracle at the float32 bar and the one-pass kernel."""
    torch = _torch()
    from mamba3_rocm import _lib
    N, P = 128, 64
    assert _lib.load().m3_chunk_scan_ws_bytes(B, L, H, N, P, R, CS, _lib.DTYPE_F32) > 0
    d = I.scan_inputs(B, L, H, N, P, R, seed=22, Hqk=Hqk, bf16=False)
    t = to_dev(d, torch.float32)
    print(f"case f32 split {(B, L, H, Hqk, R, CS)}", flush=True)
    split = hip_scan(t, CS).cpu().numpy()
    single = hip_scan(t, CS, seq_split=False).cpu().numpy()
    ref = oracle_scan(d, CS)
    print(f"  rel={rel(split, ref):.3e} vs single {rel(split, single):.3e}", flush=True)
    assert np.isfinite(split).all()
    assert rel(split, ref) <= 1e-4
    assert rel(split, single) <= 1e-4


@pytest.mark.parametrize("bf16", [True, False])
def test_sequence_split_carry_in_and_out(bf16):
    """The split path consumes an initial carry (segment 0) and returns the last
    segment's exit carry, like the one-pass kernel."""
    torch = _torch()
    from mamba3_rocm import mamba3_siso_hip_carry
    B, L, H, N, P, R = 1, 900, 2, 128, 64, 32
    L1 = 100
    d = I.scan_inputs(B, L1 + L, H, N, P, R, seed=22, bf16=bf16)
    t = to_dev(d, torch.bfloat16 if bf16 else torch.float32)
    tol = BF16_TOL if bf16 else 1e-4

    def part(lo, hi, carry, split):
        s = {k: (v[:, lo:hi] if k in ("Q", "K", "V", "Z", "Angles") else
                 v[:, :, lo:hi] if k in ("ADT", "DT", "Trap") else v) for k, v in t.items()}
        return mamba3_siso_hip_carry(s["Q"], s["K"], s["V"], s["ADT"], s["DT"], s["Trap"],
                                     s["Q_bias"], s["K_bias"], s["Angles"], s["D"], s["Z"], 64,
                                     initial_carry=carry, seq_split=split)

    _, c1 = part(0, L1, None, False)
    y_split, c_split = part(L1, L1 + L, c1, True)
    y_one, c_one = part(L1, L1 + L, c1, False)
    torch.cuda.synchronize()
    ref = oracle_scan(d, 64)[:, L1:]
    assert rel(y_split.float().cpu().numpy(), ref) <= tol
    assert rel(y_split.float().cpu().numpy(), y_one.float().cpu().numpy()) <= tol
    th_a, th_b = c_split[0].cpu().numpy(), c_one[0].cpu().numpy()
    assert rel(np.cos(th_a), np.cos(th_b)) <= 1e-4 and rel(np.sin(th_a), np.sin(th_b)) <= 1e-4
    for a, b in zip(c_split[1:], c_one[1:]):
        assert rel(a.cpu().numpy(), b.cpu().numpy()) <= (1e-2 if bf16 else 1e-4)


def test_only_one_hip_runtime_loaded():
    """The library binds to torch's HIP runtime (one libamdhip64 in the process)."""
    import os
    torch = _torch()
    from mamba3_rocm import load
    load()
    torch.zeros(1, device="cuda")
    maps = open(f"/proc/{os.getpid()}/maps").read()
    libs = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(libs) == 1, libs
