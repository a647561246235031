"""The allocation-free split prefill (m3_chunk_scan_fwd_noalloc) against the entry
point it varies (m3_chunk_scan_fwd_ws with a workspace from torch), through the C
ABI.  Both run the same kernels, so the outputs and final carries must be bitwise
equal.  Two calls in a row, the second with a smaller input (and an initial carry):
the library's scratch keeps the first call's contents, which the second must not
depend on.  Each shape takes the sequence split (B*H well below the CU count).
"""
import ctypes

import numpy as np
import pytest

from _util import I, to_dev

pytestmark = pytest.mark.gpu


def _call(lib, fn, t, out, init, fin, dims, CS, ws=None):
    import torch
    B, L, H, N, P, R = dims
    ptr = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    args = [ptr(t[k]) for k in ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")]
    args += [ptr(out)] + [ptr(x) for x in init] + [ptr(x) for x in fin]
    args += [B, L, H, H, N, P, R, CS, 1]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    args += [torch.cuda.current_stream().cuda_stream]
    rc = getattr(lib, fn)(*args)
    assert rc == 0, lib.m3_last_error().decode()


# (4, 2048, 24): 96 pairs in 8 segments, three rounds of 256 blocks and 51 MB of the
# scratch (the split's largest kind of need); the later shapes are smaller
@pytest.mark.parametrize("B,L,H,with_init", [(4, 2048, 24, False), (1, 4096, 8, False), (1, 1100, 4, True)])
def test_noalloc_equals_workspace_entry(B, L, H, with_init):
    import torch
    from mamba3_rocm import _lib
    lib = _lib.load()
    N, P, R, CS = 128, 64, 32, 64
    dims = (B, L, H, N, P, R)
    need = lib.m3_chunk_scan_ws_bytes(B, L, H, N, P, R, CS, 1)
    assert need > 0, "the shape must take the sequence split"
    d = I.scan_inputs(B, L, H, N, P, R, seed=77 + L, bf16=True)
    t = to_dev(d, torch.bfloat16)
    f32 = dict(device="cuda", dtype=torch.float32)
    g = torch.Generator(device="cuda")
    g.manual_seed(L)
    if with_init:
        init = (torch.rand(B, H, R, generator=g, **f32) * 6.0, torch.randn(B, H, P, N, generator=g, **f32) * 0.1,
                torch.randn(B, H, N, generator=g, **f32) * 0.1, torch.randn(B, H, P, generator=g, **f32))
    else:
        init = (None,) * 4
    shapes = [(B, H, R), (B, H, P, N), (B, H, N), (B, H, P)]
    outs, fins = [], []
    for fn in ("m3_chunk_scan_fwd_ws", "m3_chunk_scan_fwd_noalloc"):
        out = torch.full((B, L, H, P), float("nan"), device="cuda", dtype=torch.bfloat16)
        fin = tuple(torch.full(s, float("nan"), **f32) for s in shapes)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda") if fn == "m3_chunk_scan_fwd_ws" else None
        print(f"[noalloc] {fn} B={B} L={L} H={H} init={with_init} ws={need}", flush=True)
        _call(lib, fn, t, out, init, fin, dims, CS, ws)
        torch.cuda.synchronize()
        outs.append(out)
        fins.append(fin)
    assert torch.isfinite(outs[0].float()).all()
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(fins[0], fins[1]):
        assert torch.isfinite(a).all()
        assert torch.equal(a, b)


def test_noalloc_one_pass_shape_needs_no_scratch():
    """A shape that runs as one pass (B*H fills the chip) takes the plain kernel."""
    import torch
    from mamba3_rocm import _lib
    lib = _lib.load()
    B, L, H, N, P, R, CS = 4, 300, 64, 128, 64, 32, 64
    assert lib.m3_chunk_scan_ws_bytes(B, L, H, N, P, R, CS, 1) == 0
    d = I.scan_inputs(B, L, H, N, P, R, seed=5, bf16=True)
    t = to_dev(d, torch.bfloat16)
    outs = []
    for fn in ("m3_chunk_scan_fwd_ws", "m3_chunk_scan_fwd_noalloc"):
        out = torch.empty(B, L, H, P, device="cuda", dtype=torch.bfloat16)
        ws = torch.empty(16, dtype=torch.uint8, device="cuda") if fn == "m3_chunk_scan_fwd_ws" else None
        _call(lib, fn, t, out, (None,) * 4, (None,) * 4, (B, L, H, N, P, R), CS, ws)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    assert np.isfinite(outs[1].float().cpu().numpy()).all()
