"""m3_split_bf16x3 and the split-bf16 products of a bf16 stack's float32 head.

The parts are pinned exactly: hi equals torch's round-to-nearest-even bf16 cast of x
and lo the same cast of x - hi, in both layouts (side by side and stacked, lo in the
middle) and on both the 8-wide and the scalar path (a row length that is not a
multiple of 8).  The product a_hi b_hi + a_hi b_lo + a_lo b_hi through torch.mm with a
float32 output is checked against float64: relative error at most 2e-5 (what the
omitted a_lo b_lo and lo's rounding leave: about 2^-16 per product, observed 4e-6 at
the decoder's shape), where a float32 GEMM gives about 5e-7.
"""
import numpy as np
import pytest

from _util import rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K", [(1000, 200), (37, 13), (4, 2112)])
def test_split_parts_are_the_bf16_casts(M, K):
    import torch
    from mamba3_rocm.stack import split_bf16x3
    g = torch.Generator(device="cuda")
    g.manual_seed(M + K)
    x = torch.randn(M, K, device="cuda", generator=g) * torch.logspace(-8, 8, K, device="cuda")
    print(f"case split parts M={M} K={K}", flush=True)
    hi = x.to(torch.bfloat16)
    lo = (x - hi.float()).to(torch.bfloat16)
    s = split_bf16x3(x)
    assert torch.equal(s[:, :K], hi) and torch.equal(s[:, K:2 * K], hi) and torch.equal(s[:, 2 * K:], lo)
    r = split_bf16x3(x, stacked=True, lo_mid=True)
    assert torch.equal(r[:M], hi) and torch.equal(r[M:2 * M], lo) and torch.equal(r[2 * M:], hi)
    r = split_bf16x3(x, stacked=True)
    assert torch.equal(r[:M], hi) and torch.equal(r[M:2 * M], hi) and torch.equal(r[2 * M:], lo)
    err = ((hi.double() + lo.double() - x.double()).abs() / x.double().abs()).max().item()
    print(f"split parts: hi + lo reconstructs x to {err:.2e} relative per element", flush=True)
    assert err <= 2.0 ** -16


def test_split_product_against_float64():
    import torch
    from mamba3_rocm.stack import split_bf16x3
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    M, K, N = 4096, 768, 2112
    x = torch.randn(M, K, device="cuda", generator=g)
    w = torch.randn(N, K, device="cuda", generator=g) / K ** 0.5
    print("case split product", flush=True)
    wh = w.to(torch.bfloat16)
    wl = (w - wh.float()).to(torch.bfloat16)
    z = torch.mm(split_bf16x3(x), torch.cat([wh, wl, wh], 1).t(), out_dtype=torch.float32)
    ref = (x.double() @ w.double().t()).cpu().numpy()
    e_split = rel(z.double().cpu().numpy(), ref)
    e_f32 = rel((x @ w.t()).double().cpu().numpy(), ref)
    print(f"split product: {e_split:.2e} (float32 GEMM {e_f32:.2e})", flush=True)
    assert np.isfinite(e_split) and e_split <= 2e-5
