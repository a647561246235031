"""The C-ABI library and the host layer, without a GPU.

The library must load, export every function include/mamba3_scan.h declares,
select kernels as documented, and reject invalid calls with the documented
error codes before any device work.  The torch-facing wrappers must refuse
CPU tensors (there is no CPU fallback) and validate shapes with the
reference's messages.
"""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mamba3_scan.h")
HEADERS = [HEADER, os.path.join(ROOT, "include", "mamba3_layer.h")]


@pytest.fixture(scope="module")
def lib():
    from mamba3_rocm import _lib
    return _lib.load()


def _header_functions():
    text = "\n".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(m3_\w+)\s*\(", text, re.M)))


def _header_define(name):
    m = re.search(rf"#define\s+{name}\s+(\d+)", open(HEADER).read())
    return int(m.group(1))


def test_library_exports_every_declared_symbol(lib):
    names = _header_functions()
    assert names == sorted(["m3_abi_version", "m3_last_error", "m3_chunk_scan_impl",
                            "m3_chunk_scan_fwd", "m3_chunk_scan_fwd_carry", "m3_chunk_scan_ws_bytes",
                            "m3_chunk_scan_fwd_ws", "m3_chunk_scan_fwd_noalloc",
                            "m3_chunk_scan_bwd_ws_bytes", "m3_chunk_scan_bwd",
                            "m3_chunk_scan_fwd_shared", "m3_chunk_scan_bwd_shared_ws_bytes",
                            "m3_chunk_scan_bwd_shared", "m3_chunk_scan_saved_bytes",
                            "m3_chunk_scan_fwd_train", "m3_chunk_scan_bwd_saved_ws_bytes",
                            "m3_chunk_scan_bwd_saved", "m3_chunk_scan_fwd_train_shared",
                            "m3_chunk_scan_bwd_saved_shared_ws_bytes", "m3_chunk_scan_bwd_saved_shared",
                            "m3_decode_step", "m3_layer_pre", "m3_layer_decode_step", "m3_split_bf16x3",
                            "m3_layer_scan", "m3_layer_scan_carry", "m3_layer_scan_train", "m3_layer_scan_bwd",
                            "m3_layer_post",
                            "m3_layer_post_bwd_ws_bytes", "m3_layer_post_bwd",
                            "m3_layer_pre_bwd_ws_bytes", "m3_layer_pre_bwd", "m3_block_norm", "m3_block_gelu",
                            "m3_block_act", "m3_block_act_norm", "m3_log_softmax", "m3_block_act_bwd",
                            "m3_block_gelu_bwd", "m3_block_norm_bwd_ws_bytes", "m3_block_norm_bwd",
                            "m3_log_softmax_nll"])
    for n in names:
        assert hasattr(lib, n), n
    from mamba3_rocm import _lib
    assert sorted(_lib.EXPORTS) == names


def test_abi_version_and_constants(lib):
    from mamba3_rocm import _lib
    assert lib.m3_abi_version() == 107
    assert _lib.DTYPE_F32 == _header_define("M3_DTYPE_F32")
    assert _lib.DTYPE_BF16 == _header_define("M3_DTYPE_BF16")
    assert _lib.IMPL_CHUNKED_MFMA == _header_define("M3_IMPL_CHUNKED_MFMA")
    assert _lib.IMPL_GENERIC == _header_define("M3_IMPL_GENERIC")
    for name in ("M3_OK", "M3_E_ARG", "M3_E_ALIGN", "M3_E_UNSUPPORTED", "M3_E_LAUNCH"):
        assert getattr(_lib, name) == _header_define(name), name


def test_kernel_selection(lib):
    f = lib.m3_chunk_scan_impl
    CH, GEN, NONE = 1, 2, 0
    assert f(1, 128, 64, 32, 64) == CH          # headline bf16 shape
    assert f(1, 128, 64, 64, 64) == CH          # rope_fraction 1.0
    assert f(1, 128, 64, 32, 32) == CH          # chunk 32
    assert f(0, 64, 64, 16, 64) == CH           # fp32, config 1
    assert f(0, 128, 64, 32, 64) == CH          # fp32 at the model's geometry (d_state 128, headdim 64)
    assert f(0, 128, 64, 0, 64) == GEN          # fp32, d_state 128 without rope
    assert f(1, 128, 64, 32, 128) == CH         # chunk 128: 64-token sub-chunks
    assert f(1, 128, 64, 32, 96) == GEN         # chunk 96: no instantiation
    assert f(1, 64, 16, 16, 16) == GEN          # headdim 16
    assert f(0, 4, 4, 1, 4) == GEN              # tiny model shapes
    assert f(1, 1024, 64, 0, 64) == NONE        # state too large for either kernel
    assert f(7, 128, 64, 32, 64) == NONE        # unknown dtype


def test_split_workspace_sizes(lib):
    """Workspace for the sequence split: per (b, h, segment) two carries (P x N state,
    N key, P value, R angles, each array 256-byte aligned) and one log-decay (float32
    whatever the I/O type); none when B*H already fills the chip, for short sequences,
    or shapes without the state-only pass."""
    f = lib.m3_chunk_scan_ws_bytes
    bf, f32 = 1, 0
    al = lambda n: (n * 4 + 255) // 256 * 256  # noqa: E731
    # config 3: B*H = 32 -> 8 segments of 4096 tokens
    bhs = 32 * 8
    assert f(1, 32768, 32, 128, 64, 32, 128, bf) == (2 * (al(bhs * 64 * 128) + al(bhs * 128) + al(bhs * 64) + al(bhs * 32))
                                                     + al(bhs))
    assert f(8, 4096, 32, 128, 64, 32, 64, bf) == 0          # config 2: 256 (b, h) pairs
    assert f(1, 400, 2, 128, 64, 32, 64, bf) == 0            # too short to split
    assert f(1, 4096, 2, 128, 64, 32, 64, f32) == f(1, 4096, 2, 128, 64, 32, 64, bf) > 0   # fp32: the same carries
    assert f(1, 4096, 2, 64, 64, 16, 64, f32) == 0           # fp32 d_state 64: no state-only pass
    assert f(1, 4096, 2, 64, 64, 16, 64, bf) == 0            # no state-only pass for d_state 64
    assert f(1, 4096, 2, 128, 64, 32, 48, bf) == 0           # chunk 48: generic kernel
    assert f(1, 1061, 3, 128, 64, 32, 64, bf) > 0
    # config 5's layer: B*H = 96 -> 8 segments of 1536 tokens (768 blocks: three whole
    # rounds of 256), not 2 (192 blocks, and 96 in the state-only pass)
    assert _fwd_segments(4, 24, 12288) == (8, 1536)
    bhs = 96 * 8
    assert f(4, 12288, 24, 128, 64, 32, 64, bf) == (2 * (al(bhs * 64 * 128) + al(bhs * 128) + al(bhs * 64) + al(bhs * 32))
                                                    + al(bhs))
    assert _fwd_segments(1, 32, 32768) == (8, 4096)
    assert _fwd_segments(2, 64, 8192) == (2, 4096)     # 128 pairs: one round of 256 blocks


def test_split_workspace_fits_the_noalloc_scratch(lib):
    """m3_chunk_scan_fwd_noalloc holds 67 MiB per GPU: every split shape fits (at most
    four rounds of 256 blocks, 1024 carry slots, at d_state 128, headdim 64, R <= 64)."""
    f = lib.m3_chunk_scan_ws_bytes
    worst = 0
    for H in (1, 2, 3, 5, 8, 16, 24, 32, 48, 64, 96, 128):
        for L in (512, 1000, 2048, 4096, 12288, 32768, 100000, 1 << 20):
            worst = max(worst, f(1, L, H, 128, 64, 64, 64, 1), f(1, L, H, 128, 64, 64, 64, 0))
    assert 0 < worst <= 67 << 20
    assert f(4, 2048, 24, 128, 64, 32, 64, 1) > 17 << 20        # the no-alloc GPU test's first shape
    assert _fwd_segments(4, 24, 2048) == (8, 256)


def _fwd_segments(B, H, L):
    """(segments, tokens per segment) of the forward's sequence split, or (0, 0).
    Segments are multiples of 128 tokens, at least 256, at most four rounds of 256
    blocks.  Each block takes a fixed time per token, so n blocks of len tokens take
    ceil(n / 256) rounds of len; the state-only pass (every segment but the last) runs
    at half the full pass's time per token.  The count with the least time (the fewest
    on ties) is taken."""
    bh = B * H
    if bh * 2 > 256 or L < 512:
        return 0, 0
    best, best_cost = (0, 0), None
    for s in range(2, min(L // 256, 4 * 256 // bh) + 1):
        ln = ((L + s - 1) // s + 127) // 128 * 128
        ns = (L + ln - 1) // ln
        if ns < 2:
            continue
        cost = (2 * -(-bh * ns // 256) + -(-bh * (ns - 1) // 256)) * ln
        if best_cost is None or cost < best_cost:
            best, best_cost = (ns, ln), cost
    return best


def _walk_segments(B, H, L, cs):
    """(segments, chunks per segment) of the backward's walk (0 segments: the
    chunk-parallel route).  Split candidates: at least two segments of at least 4
    chunks, at most four rounds of 256 blocks; their time, in half-chunks of one walk
    block: 2 ceil(walk blocks / 256) seg_nc for the walk, plus ceil(adjoint blocks /
    512) chunks per adjoint block for the adjoint-only pass (sub-segments: seg_nc // 8,
    between 1 and 4, per segment but the last; two blocks per compute unit).  The count
    with the least time (the fewest on ties) is taken.  256 pairs or more: one segment;
    80 or more: the split if it takes at most 0.8 of the one-segment walk (2 nc), else
    one segment; fewer: the split if there is one, else the chunk-parallel route."""
    nc = (L + cs - 1) // cs
    bh = B * H
    if bh >= 256:
        return 1, nc
    best, best_cost = None, None
    for s in range(2, min(nc // 4, 4 * 256 // bh) + 1):
        seg_nc = (nc + s - 1) // s
        ns = (nc + seg_nc - 1) // seg_nc
        if ns < 2:
            continue
        sub = max(1, min(4, seg_nc // 8))
        cost = 2 * -(-bh * ns // 256) * seg_nc + -(-bh * (ns - 1) * sub // 512) * -(-seg_nc // sub)
        if best_cost is None or cost < best_cost:
            best, best_cost = (ns, seg_nc), cost
    if bh >= 80:
        return best if best is not None and 10 * best_cost <= 16 * nc else (1, nc)
    return best if best is not None else (0, nc)


def _split_ws(B, H, L, N, P, R):
    """The sequence split's carries (test_split_workspace_sizes): two sets per
    (b, h, segment) and one log-decay; 0 without a split."""
    al = lambda n: (n * 4 + 255) // 256 * 256  # noqa: E731
    nseg, _ = _fwd_segments(B, H, L)
    if nseg < 2 or N != 128 or P != 64:
        return 0
    bhs = B * H * nseg
    return 2 * (al(bhs * P * N) + al(bhs * N) + al(bhs * P) + al(bhs * max(R, 1))) + al(bhs)


def _bwd_ws_expect(B, L, H, Hqk, N, P, R, io, saved=False):
    """Backward workspace: chunk-entering states (B*H*nc*P*N in the I/O type, 64-token
    chunks for bf16, 32 for fp32) and chunk angles (unless the training forward saved
    them), adjoint states after each chunk (chunk-parallel route only), bias and D
    partials, per-token d(scale), chunk sums of dA and d(theta), per-head dQ/dK
    (in the I/O type) when Hqk < H, the split walk's segment adjoints (two float32 P x N
    states per (b, h, segment) of the walk or of the adjoint pass's sub-segments, and a
    log-decay per sub-segment) and the split state pass's carries."""
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    cs = 64 if io == 1 else 32
    bhc = B * H * ((L + cs - 1) // cs)
    ts = 2 if io == 1 else 4
    nseg, seg_nc = _walk_segments(B, H, L, cs)
    sub = max(1, min(4, seg_nc // 8))          # the adjoint pass's sub-segments per segment
    n = 2 * al(bhc * N * 4) + al(bhc * 4) + al(B * H * L * 4) + al(bhc * (R + 1) * 4)
    if not saved:
        n += al(bhc * P * N * ts) + al(bhc * max(R, 1) * 4)
    if nseg == 0:
        n += al(bhc * P * N * ts)
    if Hqk < H:
        n += 2 * al(B * L * H * N * ts)
    if nseg > 1:
        n += al(B * H * nseg * P * N * 4) + al(B * H * nseg * sub * P * N * 4) + al(B * H * nseg * sub * 4)
    if not saved:
        n += _split_ws(B, H, L, N, P, R)
    return n


def test_backward_workspace_sizes(lib, monkeypatch):
    monkeypatch.delenv("M3_BWD_ROUTE", raising=False)
    f = lib.m3_chunk_scan_bwd_ws_bytes
    bf, f32 = 1, 0
    assert f(8, 4096, 32, 32, 128, 64, 32, 64, bf) == _bwd_ws_expect(8, 4096, 32, 32, 128, 64, 32, bf)
    assert f(2, 300, 4, 2, 64, 32, 16, 64, f32) == _bwd_ws_expect(2, 300, 4, 2, 64, 32, 16, f32)
    # float32 at the model's geometry (what Mamba3SSM hands its scan): the walk, and
    # for few pairs the split walk and split state pass
    for B, H in ((8, 32), (1, 4)):
        for R in (32, 64):
            assert f(B, 4096, H, H, 128, 64, R, 64, f32) == _bwd_ws_expect(B, 4096, H, H, 128, 64, R, f32)
    # config 3's shape: 8 walk segments of 64 chunks (the adjoint pass in 32 sub-segments
    # of 16), 8 state-pass segments of 4096 tokens
    assert _walk_segments(1, 32, 32768, 64) == (8, 64)
    # config 5's layer (96 pairs, 192 chunks): 8 segments of 24 chunks (three rounds of
    # 256 blocks) instead of the one-segment walk on 96 compute units; 128 pairs at
    # L=4096: two segments of 32 chunks; 160 pairs: the one-segment walk
    assert _walk_segments(4, 24, 12288, 64) == (8, 24)
    assert _walk_segments(4, 32, 4096, 64) == (2, 32)
    assert _walk_segments(5, 32, 4096, 64) == (1, 64)
    assert f(4, 12288, 24, 24, 128, 64, 32, 64, bf) == _bwd_ws_expect(4, 12288, 24, 24, 128, 64, 32, bf)
    assert f(4, 4096, 32, 32, 128, 64, 32, 64, bf) == _bwd_ws_expect(4, 4096, 32, 32, 128, 64, 32, bf)
    assert f(5, 4096, 32, 32, 128, 64, 32, 64, bf) == _bwd_ws_expect(5, 4096, 32, 32, 128, 64, 32, bf)
    assert f(1, 32768, 32, 32, 128, 64, 32, 128, bf) == _bwd_ws_expect(1, 32768, 32, 32, 128, 64, 32, bf)
    assert f(1, 200, 2, 2, 128, 64, 32, 64, bf) == _bwd_ws_expect(1, 200, 2, 2, 128, 64, 32, bf)  # chunks
    assert f(1, 100, 2, 2, 64, 16, 16, 64, bf) == 0        # headdim 16: no backward kernel
    assert f(1, 100, 2, 2, 128, 64, 32, 64, 7) == 0        # unknown dtype
    assert f(1, 100, 3, 2, 128, 64, 32, 64, bf) == 0       # H not a multiple of Hqk
    # the route can be forced (the chunk-parallel route adds the adjoint states)
    monkeypatch.setenv("M3_BWD_ROUTE", "chunks")
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    assert f(8, 4096, 32, 32, 128, 64, 32, 64, bf) == (_bwd_ws_expect(8, 4096, 32, 32, 128, 64, 32, bf)
                                                        + al(8 * 32 * 64 * 64 * 128 * 2))


def test_saved_state_sizes_and_validation(lib, monkeypatch):
    """The training pair: the residual buffer holds the chunk-entering states (io type)
    and chunk angles (float32) of the backward's chunking and the output before the
    gate (float32 I/O only, B x L x H x P); the saved-state backward's workspace
    drops the states; calls validate before any launch."""
    monkeypatch.delenv("M3_BWD_ROUTE", raising=False)
    E_ARG, E_UNSUP = _header_define("M3_E_ARG"), _header_define("M3_E_UNSUPPORTED")
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    bf, f32 = 1, 0
    sb = lib.m3_chunk_scan_saved_bytes
    assert sb(8, 4096, 32, 128, 64, 32, bf) == al(8 * 32 * 64 * 64 * 128 * 2) + al(8 * 32 * 64 * 32 * 4)
    assert sb(2, 300, 4, 64, 32, 16, f32) == (al(2 * 4 * 10 * 32 * 64 * 4) + al(2 * 4 * 10 * 16 * 4)
                                              + al(2 * 300 * 4 * 32 * 4))
    assert sb(8, 4096, 32, 128, 64, 32, f32) == (al(8 * 32 * 128 * 64 * 128 * 4) + al(8 * 32 * 128 * 32 * 4)
                                                + al(8 * 4096 * 32 * 64 * 4))
    assert sb(1, 100, 2, 64, 16, 16, bf) == 0               # no backward kernel
    wsb = lib.m3_chunk_scan_bwd_saved_ws_bytes
    assert wsb(8, 4096, 32, 32, 128, 64, 32, 64, bf) == _bwd_ws_expect(8, 4096, 32, 32, 128, 64, 32, bf, True)
    assert wsb(2, 300, 4, 2, 64, 32, 16, 64, f32) == _bwd_ws_expect(2, 300, 4, 2, 64, 32, 16, f32, True)
    assert wsb(8, 4096, 32, 32, 128, 64, 32, 64, f32) == _bwd_ws_expect(8, 4096, 32, 32, 128, 64, 32, f32, True)
    p = ctypes.c_void_p(4096)

    def fwd(saved=p, nbytes=1 << 40, CS=64, N=128, P=64, R=32, io=bf):
        return lib.m3_chunk_scan_fwd_train(p, p, p, p, p, p, p, p, p, p, p, p, 1, 8, 2, 2, N, P, R, CS, io,
                                           saved, nbytes, None, 0, None)
    assert fwd(saved=None) == E_ARG
    assert fwd(nbytes=16) == E_ARG and b"saved-state buffer" in lib.m3_last_error()
    assert fwd(CS=32) == E_UNSUP and b"multiple of 64" in lib.m3_last_error()
    assert fwd(P=16) == E_UNSUP                              # no backward for the shape
    assert fwd(io=f32, CS=48, N=64, P=64, R=16) == E_UNSUP   # f32: multiple of 32

    def bwd(saved=p, nbytes=1 << 40):
        return lib.m3_chunk_scan_bwd_saved(p, p, p, p, p, p, p, p, p, p, p, p,
                                           p, p, p, p, p, p, p, p, p, p, p,
                                           1, 8, 2, 2, 128, 64, 32, 64, bf, saved, nbytes, p, 1 << 40, None)
    assert bwd(saved=None) == E_ARG
    assert bwd(nbytes=16) == E_ARG and b"saved-state buffer" in lib.m3_last_error()


def test_backward_validation(lib):
    E_ARG, E_UNSUP = _header_define("M3_E_ARG"), _header_define("M3_E_UNSUPPORTED")
    p = ctypes.c_void_p(4096)

    def call(Z=p, dZ=p, N=128, P=64, R=32, ws=p, wsb=1 << 40, **kw):
        d = dict(B=1, L=8, H=2, Hqk=2, io=1)
        d.update(kw)
        return lib.m3_chunk_scan_bwd(p, p, p, p, p, p, p, p, p, p, Z, p,
                                     p, p, p, p, p, p, p, p, p, p, dZ,
                                     d["B"], d["L"], d["H"], d["Hqk"], N, P, R, 64, d["io"], ws, wsb, None)
    assert call(P=16) == E_UNSUP and b"no backward kernel" in lib.m3_last_error()
    assert call(Z=None) == E_ARG and b"dZ" in lib.m3_last_error()
    assert call(ws=None) == E_ARG and b"workspace" in lib.m3_last_error()
    assert call(wsb=16) == E_ARG
    assert call(H=3) == E_ARG
    assert call(B=0) == 0


def _scan_call(lib, **kw):
    a = dict(Q=None, K=None, V=None, ADT=None, DT=None, Trap=None, Qb=None, Kb=None, Ang=None,
             D=None, Z=None, Out=None, B=1, L=8, H=2, Hqk=2, N=64, P=64, R=16, CS=64, io=1)
    a.update(kw)
    return lib.m3_chunk_scan_fwd(a["Q"], a["K"], a["V"], a["ADT"], a["DT"], a["Trap"], a["Qb"],
                                 a["Kb"], a["Ang"], a["D"], a["Z"], a["Out"], a["B"], a["L"], a["H"],
                                 a["Hqk"], a["N"], a["P"], a["R"], a["CS"], a["io"], None)


def test_validation_errors_before_any_launch(lib):
    E_ARG, E_UNSUP = _header_define("M3_E_ARG"), _header_define("M3_E_UNSUPPORTED")
    assert _scan_call(lib, io=5) == E_ARG
    assert b"io_dtype" in lib.m3_last_error()
    assert _scan_call(lib, H=3, Hqk=2) == E_ARG
    assert b"divisible by nheads_qk" in lib.m3_last_error()
    assert _scan_call(lib, R=40) == E_ARG
    assert b"<= d_state/2" in lib.m3_last_error()
    assert _scan_call(lib, N=0) == E_ARG
    assert _scan_call(lib) == E_ARG                      # NULL required pointers
    assert b"NULL" in lib.m3_last_error()
    assert _scan_call(lib, B=0) == 0                     # empty batch is a no-op
    assert _scan_call(lib, L=0) == 0
    assert lib.m3_last_error() == b""
    fake = ctypes.c_void_p(4096)                         # never dereferenced: rejected first
    assert _scan_call(lib, Q=fake, K=fake, V=fake, ADT=fake, DT=fake, Trap=fake, Qb=fake, Kb=fake,
                      Ang=fake, Out=fake, N=1024, P=64, R=0) == E_UNSUP


def test_misaligned_pointer_rejected(lib):
    E_ALIGN = _header_define("M3_E_ALIGN")
    ok = ctypes.c_void_p(4096)
    bad = ctypes.c_void_p(4098)
    assert _scan_call(lib, Q=bad, K=ok, V=ok, ADT=ok, DT=ok, Trap=ok, Qb=ok, Kb=ok, Ang=ok,
                      Out=ok) == E_ALIGN


def test_backward_misaligned_angle_gradient_rejected(lib):
    """The backward stores dAngles and reads Angles as 16-byte pieces: a misaligned
    pointer is refused before any launch."""
    E_ALIGN = _header_define("M3_E_ALIGN")
    ok, bad = ctypes.c_void_p(4096), ctypes.c_void_p(4100)
    ws = lib.m3_chunk_scan_bwd_ws_bytes(1, 128, 2, 2, 128, 64, 32, 64, 1)
    for ang, dang in ((bad, ok), (ok, bad)):
        args = [ok] * 8 + [ang] + [ok] * 3 + [ok] * 8 + [dang] + [ok, ok]
        rc = lib.m3_chunk_scan_bwd(*args, 1, 128, 2, 2, 128, 64, 32, 64, 1, ok, ws, None)
        assert rc == E_ALIGN and b"16-byte aligned" in lib.m3_last_error()


def test_carry_arguments_all_or_none(lib):
    p = ctypes.c_void_p(4096)
    rc = lib.m3_chunk_scan_fwd_carry(p, p, p, p, p, p, p, p, p, None, None, p,
                                     p, None, None, None, None, None, None, None,
                                     1, 8, 2, 2, 64, 64, 16, 64, 1, None)
    assert rc == _header_define("M3_E_ARG")
    assert b"initial carry" in lib.m3_last_error()


def test_decode_validation(lib):
    E_ARG, E_UNSUP = _header_define("M3_E_ARG"), _header_define("M3_E_UNSUPPORTED")
    p = ctypes.c_void_p(4096)
    args = [p] * 16

    def call(**kw):
        d = dict(B=2, H=2, N=64, P=32, R=16, ind=1, outd=0, am=1, dm=0)
        d.update(kw)
        return lib.m3_decode_step(*args, d["B"], d["H"], d["N"], d["P"], d["R"], d["ind"], d["outd"],
                                  d["am"], d["dm"], None)
    assert call(am=2) == E_ARG and b"angle_mode" in lib.m3_last_error()
    assert call(dm=3) == E_ARG and b"diag_mode" in lib.m3_last_error()
    assert call(R=33) == E_ARG
    assert call(N=12, R=4) == E_UNSUP                   # d_state/4 not a power of two
    assert call(B=0) == 0


def test_layer_decode_validation(lib):
    E_ARG, E_UNSUP = _header_define("M3_E_ARG"), _header_define("M3_E_UNSUPPORTED")
    p = ctypes.c_void_p(4096)

    def call(ptrs=None, **kw):
        d = dict(B=2, H=2, P=32, N=64, R=16, io=1, am=1, dm=0)
        d.update(kw)
        return lib.m3_layer_decode_step(*(ptrs or [p] * 12), d["B"], d["H"], d["P"], d["N"], d["R"], 1e-4, 1e-6,
                                        d["io"], d["am"], d["dm"], None)
    assert call(io=7) == E_ARG and b"io_dtype" in lib.m3_last_error()
    assert call(am=2) == E_ARG and b"angle_mode" in lib.m3_last_error()
    assert call(dm=3) == E_ARG and b"diag_mode" in lib.m3_last_error()
    assert call(R=33) == E_ARG
    assert call(H=0) == E_ARG
    assert call(N=12, R=4) == E_UNSUP                   # d_state/4 not a power of two
    assert call(ptrs=[None] + [p] * 11) == E_ARG and b"NULL" in lib.m3_last_error()
    assert call(ptrs=[p] * 8 + [ctypes.c_void_p(4100)] + [p] * 3) == _header_define("M3_E_ALIGN")
    assert call(B=0) == 0


def test_split_bf16x3_validation(lib):
    E_ARG = _header_define("M3_E_ARG")
    p = ctypes.c_void_p(4096)
    assert lib.m3_split_bf16x3(p, p, None, p, -1, 8, 8, None) == E_ARG
    assert lib.m3_split_bf16x3(p, p, None, p, 4, 0, 8, None) == E_ARG
    assert lib.m3_split_bf16x3(p, p, None, p, 4, 8, 7, None) == E_ARG and b"stride" in lib.m3_last_error()
    assert lib.m3_split_bf16x3(None, p, None, p, 4, 8, 8, None) == E_ARG and b"NULL" in lib.m3_last_error()
    assert lib.m3_split_bf16x3(p, p, p, None, 4, 8, 8, None) == E_ARG
    assert lib.m3_split_bf16x3(p, p, None, p, 0, 8, 8, None) == 0


def test_wrappers_refuse_cpu_tensors():
    import torch
    from mamba3_rocm import mamba3_siso_hip, rnn_step_hip
    L, H, N, P, R = 8, 2, 64, 32, 16
    z = lambda *s: torch.zeros(*s)  # noqa: E731
    with pytest.raises(ValueError, match="ROCm device tensor"):
        mamba3_siso_hip(z(L, H, N), z(L, H, N), z(L, H, P), z(H, L), z(H, L), z(H, L), z(H, N),
                        z(H, N), z(L, H, R), z(H), z(L, H, P), 64)
    carry = (z(1, H, R), z(1, H, P, N), z(1, H, N), z(1, H, P))
    tin = (z(1, H, P), z(1, H, P), z(1, H, N), z(1, H, N), z(1, H), z(1, H), z(1, H), z(1, H, R))
    with pytest.raises(ValueError, match="ROCm device tensor"):
        rnn_step_hip(carry, tin, z(H, N), z(H, N), z(H))


def test_mode_knobs_match_reference(monkeypatch):
    from mamba3_rocm import recurrent_angle_mode, recurrent_diagonal_mode
    monkeypatch.delenv("MAMBA3_RECURRENT_DIAGONAL_MODE", raising=False)
    monkeypatch.delenv("MAMBA3_RECURRENT_ANGLE_MODE", raising=False)
    assert recurrent_diagonal_mode() == "current"
    assert recurrent_angle_mode() == "wrapped"
    monkeypatch.setenv("MAMBA3_RECURRENT_DIAGONAL_MODE", "legacy_double")
    monkeypatch.setenv("MAMBA3_RECURRENT_ANGLE_MODE", "legacy_unbounded")
    assert recurrent_diagonal_mode() == "legacy_double"
    assert recurrent_angle_mode() == "legacy_unbounded"
    monkeypatch.setenv("MAMBA3_RECURRENT_DIAGONAL_MODE", "x")
    with pytest.raises(ValueError, match="MAMBA3_RECURRENT_DIAGONAL_MODE"):
        recurrent_diagonal_mode()
    monkeypatch.setenv("MAMBA3_RECURRENT_ANGLE_MODE", "x")
    with pytest.raises(ValueError, match="MAMBA3_RECURRENT_ANGLE_MODE"):
        recurrent_angle_mode()


def test_bench_byte_and_flop_formulas():
    """bench.py's algorithmic counts at config 2 and config 4."""
    import bench
    assert bench.scan_bytes(8, 4096, 32, 128, 64, 32, 2) == 8 * 4096 * 32 * 1036
    assert bench.scan_flops(8, 4096, 32, 128, 64, 64) == 8 * 4096 * 32 * 57344
    # f32 carry traffic + bf16 step inputs + f32 y (the reference returns y in f32)
    assert bench.decode_bytes(512, 32, 128, 64, 32, 2, 4) == 512 * 32 * 68492
    assert abs(bench.scan_bytes(8, 4096, 32, 128, 64, 32, 2) / 8e12 * 1e6 - 135.8) < 0.1
    # backward: 1944 B per token-head with bf16 I/O, 3608 with float32; float32 MFMA work
    # per 32-token chunk-head: S, dq~, dk~ intra (3 CS^2 N), dP, y, dV intra (3 CS^2 P),
    # and five CS N P products, two FLOPs per MAC
    assert bench.bwd_bytes(8, 4096, 32, 128, 64, 32, 2) == 8 * 4096 * 32 * 1944
    assert bench.bwd_bytes(8, 4096, 32, 128, 64, 32, 4) == 8 * 4096 * 32 * 3608
    CS, N, P = 32, 128, 64
    per_chunk = 2 * (3 * CS * CS * N + 3 * CS * CS * P + 5 * CS * N * P)
    assert bench.bwd_flops(8, 4096, 32, N, P, CS) * CS == 8 * 4096 * 32 * per_chunk


def test_bf16_rounding_matches_torch():
    import torch
    from oracle import inputs as I
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 10
    ours = I.bf16_round(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours, theirs)


def test_layer_scan_validation(lib):
    """m3_layer_scan (x and z read in place from the projection) rejects bad
    arguments before any launch: dtype, a projection row that is not exactly its
    fields' width (the layout m3_layer_pre reads), rows that are not a multiple of 16
    bytes, NULL; m3_layer_pre takes V and Z together."""
    from mamba3_rocm import _lib
    fake = 1 << 20                      # never dereferenced: every call fails validation first
    H, N, P, R = 4, 128, 64, 32
    full = 2 * H * P + 2 * N + 3 * H + R      # 812 elements: 1624 bytes in bf16, not a multiple of 16

    def scan(proj, d_in_proj, io=_lib.DTYPE_BF16, heads=H):
        return lib.m3_layer_scan(fake, fake, proj, d_in_proj, fake, fake, fake, fake, fake, fake, fake, fake,
                                 2, 64, heads, N, P, R, 64, io, None, 0, None)
    assert scan(fake, full, io=7) == _lib.M3_E_ARG
    assert scan(fake, full - 1) == _lib.M3_E_ARG
    assert scan(fake, full + 4) == _lib.M3_E_ARG          # padded rows: m3_layer_pre reads the exact width
    assert b"width" in lib.m3_last_error()
    assert scan(fake, full) == _lib.M3_E_ALIGN
    assert b"16" in lib.m3_last_error()
    full8 = 2 * 8 * P + 2 * N + 3 * 8 + R     # 1336 elements: 16-byte rows in bf16
    assert scan(None, full8, heads=8) == _lib.M3_E_ARG
    assert lib.m3_layer_pre(fake, fake, fake, fake, fake, fake, fake, None, fake, fake, fake, fake,
                            2, 64, H, P, N, R, 1e-4, 1e-6, _lib.DTYPE_BF16, None) == _lib.M3_E_ARG
    # the training pair in place: the same layout checks, for d_proj too, and the residuals
    tr = lambda proj, d_in, saved, io=_lib.DTYPE_BF16, heads=H: lib.m3_layer_scan_train(  # noqa: E731
        fake, fake, proj, d_in, fake, fake, fake, fake, fake, fake, fake, fake, 2, 64, heads, N, P, R, 64, io,
        saved, 1 << 20, None, 0, None)
    assert tr(fake, full, fake, io=7) == _lib.M3_E_ARG
    assert tr(fake, full + 8, fake) == _lib.M3_E_ARG
    assert tr(fake, full, fake) == _lib.M3_E_ALIGN
    assert tr(fake, full8, None, heads=8) == _lib.M3_E_ARG and b"saved" in lib.m3_last_error()

    def bw(proj, dproj, d_in, heads=H):
        return lib.m3_layer_scan_bwd(fake, fake, proj, d_in, fake, fake, fake, fake, fake, fake, fake, fake,
                                     fake, fake, dproj, fake, fake, fake, fake, fake, fake, fake,
                                     2, 64, heads, N, P, R, 64, _lib.DTYPE_BF16, None, 0, fake, 1 << 30, None)
    assert bw(fake, fake, full - 2) == _lib.M3_E_ARG
    assert bw(fake, fake, full) == _lib.M3_E_ALIGN
    assert bw(fake, None, full8, heads=8) == _lib.M3_E_ARG
    assert bw(None, fake, full8, heads=8) == _lib.M3_E_ARG


def test_layer_backward_entry_points_validate(lib):
    """m3_layer_post_bwd and m3_layer_pre_bwd reject bad dtypes, dimensions, shapes
    above their limits, NULL pointers, short workspaces and (post) misaligned rows
    before any launch; an empty batch is a no-op; the workspace sizes are 0 for
    non-positive dimensions and grow with the row count and the columns."""
    from mamba3_rocm import _lib
    fake = 1 << 20                      # never dereferenced: every call fails validation or is empty
    bf, f32 = _lib.DTYPE_BF16, _lib.DTYPE_F32
    B, L, D = 2, 64, 256
    ws = lib.m3_layer_post_bwd_ws_bytes(B, L, D)
    assert ws > 0 and ws % (4 * D) == 0
    assert lib.m3_layer_post_bwd_ws_bytes(0, L, D) == 0 and lib.m3_layer_post_bwd_ws_bytes(B, L, 0) == 0
    assert lib.m3_layer_post_bwd_ws_bytes(B, 4 * L, D) > ws
    assert lib.m3_layer_post_bwd_ws_bytes(B, L, 2 * D) == 2 * ws

    def post(y=fake, dn=fake, sc=fake, dy=fake, dsc=fake, B=B, L=L, D=D, io=bf, w=fake, wsb=ws):
        return lib.m3_layer_post_bwd(y, dn, sc, dy, dsc, B, L, D, 1e-6, io, w, wsb, None)
    assert post(io=9) == _lib.M3_E_ARG
    assert post(D=0) == _lib.M3_E_ARG
    assert post(D=260) == _lib.M3_E_UNSUPPORTED                    # not a multiple of 8
    assert post(D=4096, wsb=1 << 30) == _lib.M3_E_UNSUPPORTED       # above 2048
    assert post(B=0, y=None) == _lib.M3_OK
    assert post(dsc=None) == _lib.M3_E_ARG
    assert post(w=None) == _lib.M3_E_ARG
    assert post(wsb=ws - 4) == _lib.M3_E_ARG and b"workspace" in lib.m3_last_error()
    assert post(dy=fake + 8) == _lib.M3_E_ALIGN
    assert post(D=8, io=f32, wsb=lib.m3_layer_post_bwd_ws_bytes(B, L, 8), dy=None) == _lib.M3_E_ARG

    H, P, N, R = 4, 64, 128, 32
    wsp = lib.m3_layer_pre_bwd_ws_bytes(B, L, H, N)
    assert wsp > 0 and wsp % (4 * (2 * N + H)) == 0
    assert lib.m3_layer_pre_bwd_ws_bytes(B, L, 0, N) == 0 and lib.m3_layer_pre_bwd_ws_bytes(B, 0, H, N) == 0
    assert lib.m3_layer_pre_bwd_ws_bytes(B, 4 * L, H, N) > wsp

    def pre(proj=fake, dang=fake, dproj=fake, B=B, L=L, H=H, N=N, R=R, io=bf, w=fake, wsb=wsp):
        return lib.m3_layer_pre_bwd(proj, fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, dang, dproj,
                                    fake, fake, fake, B, L, H, P, N, R, 1e-4, 1e-6, io, w, wsb, None)
    assert pre(io=3) == _lib.M3_E_ARG
    assert pre(H=0) == _lib.M3_E_ARG
    assert pre(N=512, wsb=1 << 30) == _lib.M3_E_UNSUPPORTED and b"d_state" in lib.m3_last_error()
    assert pre(B=0, proj=None) == _lib.M3_OK
    assert pre(proj=None) == _lib.M3_E_ARG
    assert pre(dang=None) == _lib.M3_E_ARG                         # R > 0 needs dAngles
    assert pre(w=None) == _lib.M3_E_ARG
    assert pre(wsb=wsp - 4) == _lib.M3_E_ARG and b"workspace" in lib.m3_last_error()
    one_of = lib.m3_layer_pre_bwd(fake, fake, fake, fake, fake, fake, None, fake, fake, fake, fake, fake, fake,
                                  fake, fake, fake, B, L, H, P, N, R, 1e-4, 1e-6, bf, fake, wsp, None)
    assert one_of == _lib.M3_E_ARG and b"together" in lib.m3_last_error()


def test_block_entry_points_validate(lib):
    """The backbone block's C entry points (LayerNorm, gelu, activation epilogue)
    reject bad dtypes, activations and missing Dense outputs before any launch, and
    an empty batch is a no-op; the activation codes match the header."""
    from mamba3_rocm import _lib
    text = open(os.path.join(ROOT, "include", "mamba3_layer.h")).read()
    for name in ("M3_ACT_GELU", "M3_ACT_FULL_GLU", "M3_ACT_HALF_GLU1", "M3_ACT_HALF_GLU2"):
        assert getattr(_lib, name) == int(re.search(rf"#define\s+{name}\s+(\d+)", text).group(1)), name
    fake = 1 << 20                      # never dereferenced: every call fails validation or is empty
    bf = _lib.DTYPE_BF16
    assert lib.m3_block_norm(fake, fake, fake, fake, 2, 8, 64, 1e-6, 5, None) == _lib.M3_E_ARG
    assert lib.m3_block_norm(fake, None, fake, fake, 2, 8, 64, 1e-6, bf, None) == _lib.M3_E_ARG
    assert lib.m3_block_norm(fake, fake, fake, fake, 0, 8, 64, 1e-6, bf, None) == _lib.M3_OK
    assert lib.m3_block_gelu(fake, fake, 2, 8, 0, bf, None) == _lib.M3_E_ARG
    assert lib.m3_block_gelu(fake, fake, 2, 8, 64, 9, None) == _lib.M3_E_ARG
    assert lib.m3_block_act(fake, None, fake, fake, fake, 2, 8, 64, 4, bf, None) == _lib.M3_E_ARG
    assert lib.m3_block_act(fake, None, fake, fake, fake, 2, 8, 64, _lib.M3_ACT_FULL_GLU, bf, None) == _lib.M3_E_ARG
    assert b"h1" in lib.m3_last_error()
    assert lib.m3_block_act(fake, None, None, fake, fake, 2, 8, 64, _lib.M3_ACT_HALF_GLU2, bf, None) == _lib.M3_E_ARG
    assert lib.m3_block_act(fake, None, None, None, fake, 2, 8, 64, _lib.M3_ACT_GELU, bf, None) == _lib.M3_E_ARG
    assert lib.m3_block_act(fake, None, None, fake, fake, 0, 8, 64, _lib.M3_ACT_GELU, bf, None) == _lib.M3_OK
    an = lambda *a: lib.m3_block_act_norm(*a)   # noqa: E731
    assert an(fake, None, fake, fake, fake, fake, fake, fake, 2, 8, 64, 1e-6, 2, bf, 7, None) == _lib.M3_E_ARG
    assert an(fake, None, fake, fake, fake, None, fake, fake, 2, 8, 64, 1e-6, 2, bf, bf, None) == _lib.M3_E_ARG
    assert an(fake, None, fake, 4096, None, fake, fake, 4096, 2, 8, 64, 1e-6, 2, bf, bf, None) == _lib.M3_E_ARG
    assert b"alias" in lib.m3_last_error()
    assert an(fake, None, fake, fake, None, fake, fake, 4096, 0, 8, 64, 1e-6, 2, bf, bf, None) == _lib.M3_OK


def test_contraction_precision_knob(monkeypatch):
    """MAMBA3_CONTRACTION_PRECISION follows the reference's contract
    (mamba3_jax.py:44-52): highest by default (also when empty), default accepted,
    anything else raises its ValueError -- at the entry points too, before any
    device work."""
    import torch
    from mamba3_rocm import mamba3_contraction_precision_mode, mamba3_siso_hip, rnn_step_hip
    monkeypatch.delenv("MAMBA3_CONTRACTION_PRECISION", raising=False)
    assert mamba3_contraction_precision_mode() == "highest"
    monkeypatch.setenv("MAMBA3_CONTRACTION_PRECISION", "")
    assert mamba3_contraction_precision_mode() == "highest"
    monkeypatch.setenv("MAMBA3_CONTRACTION_PRECISION", "default")
    assert mamba3_contraction_precision_mode() == "default"
    for bad in ("tf32", "HIGHEST", "high"):
        monkeypatch.setenv("MAMBA3_CONTRACTION_PRECISION", bad)
        with pytest.raises(ValueError, match="MAMBA3_CONTRACTION_PRECISION must be highest or default"):
            mamba3_contraction_precision_mode()
        t = torch.zeros(1)
        with pytest.raises(ValueError, match="MAMBA3_CONTRACTION_PRECISION must be highest or default"):
            mamba3_siso_hip(t, t, torch.zeros(4, 2, 8), t, t, t, t, t, t)
        with pytest.raises(ValueError, match="MAMBA3_CONTRACTION_PRECISION must be highest or default"):
            rnn_step_hip((t, t, t, t), (t,) * 8, t, t, t)


def test_pallas_dtype_knob(monkeypatch):
    """MAMBA3_PALLAS_DTYPE follows the reference's contract (mamba3_pallas.py:112-122):
    unset or empty, the layer's dtype decides; "float32" / "bfloat16" override it;
    anything else raises its ValueError -- at the shared-B/C entry point too, before
    any device work."""
    import torch
    from mamba3_rocm import mamba3_ssd_chunked_shared_hip, pallas_compute_dtype
    monkeypatch.delenv("MAMBA3_PALLAS_DTYPE", raising=False)
    assert pallas_compute_dtype() == torch.float32
    assert pallas_compute_dtype(torch.bfloat16) == torch.bfloat16
    monkeypatch.setenv("MAMBA3_PALLAS_DTYPE", "")
    assert pallas_compute_dtype(torch.bfloat16) == torch.bfloat16
    monkeypatch.setenv("MAMBA3_PALLAS_DTYPE", "float32")
    assert pallas_compute_dtype(torch.bfloat16) == torch.float32
    monkeypatch.setenv("MAMBA3_PALLAS_DTYPE", "bfloat16")
    assert pallas_compute_dtype(torch.float32) == torch.bfloat16
    for bad in ("fp32", "bf16", "float16", "BFLOAT16"):
        monkeypatch.setenv("MAMBA3_PALLAS_DTYPE", bad)
        with pytest.raises(ValueError, match="MAMBA3_PALLAS_DTYPE must be float32 or bfloat16"):
            pallas_compute_dtype()
        t = torch.zeros(1)
        with pytest.raises(ValueError, match="MAMBA3_PALLAS_DTYPE must be float32 or bfloat16"):
            mamba3_ssd_chunked_shared_hip(t, t, torch.zeros(4, 2, 8), t, t, t, t, t, t)


def test_split_bf16x3_wrapper_refuses_other_tensors():
    import torch
    from mamba3_rocm.stack import split_bf16x3
    for bad in (torch.zeros(4, 8), torch.zeros(4, 8, dtype=torch.bfloat16), torch.zeros(2, 4, 8)):
        with pytest.raises(ValueError, match="contiguous 2-D float32 device tensor"):
            split_bf16x3(bad)
