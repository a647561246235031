"""Shared helpers for the tests (inputs, error metric, oracle calls)."""
from __future__ import annotations

import numpy as np

from oracle import inputs as I
from oracle import mamba3_ref as M

ARG_ORDER = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")


def rel(a, b):
    """The reference's error metric: max|a-b| / max|b| (test_mamba3_pallas_ssd.py:79-82)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-12))


def oracle_scan(d, chunk_size, heads=None, dtype=np.float64, no_d=False, no_z=False):
    """Batched oracle on an inputs dict from oracle.inputs.scan_inputs."""
    return M.mamba3_ssd_chunked_batched(
        d["Q"], d["K"], d["V"], d["ADT"], d["DT"], d["Trap"], d["Angles"], d["Q_bias"],
        d["K_bias"], None if no_d else d["D"], None if no_z else d["Z"],
        chunk_size=chunk_size, dtype=dtype, heads=heads)


def to_dev(d, io_dtype, device="cuda"):
    """Torch tensors on the device: Q, K, V, Z in io_dtype, the rest float32."""
    import torch
    out = {}
    for k, v in d.items():
        t = torch.from_numpy(np.ascontiguousarray(v))
        if k in ("Q", "K", "V", "Z"):
            t = t.to(io_dtype)
        out[k] = t.to(device)
    return out


def hip_scan(t, chunk_size, no_d=False, no_z=False, seq_split=True):
    from mamba3_rocm import mamba3_siso_hip
    return mamba3_siso_hip(t["Q"], t["K"], t["V"], t["ADT"], t["DT"], t["Trap"], t["Q_bias"],
                           t["K_bias"], t["Angles"], None if no_d else t["D"],
                           None if no_z else t["Z"], chunk_size, seq_split=seq_split)


def device_scan_inputs(B, L, H, N, P, R, seed, io_dtype):
    """Seeded scan inputs generated on the device (for sizes where numpy generation
    is slow), with the configurations' distributions: x, z ~ N(0,1);
    dt = softplus(N(-2, 0.5)); A_h = -exp(U[0, ln 16]); B, C and the biases
    ~ N(0,1)/sqrt(N); D ~ N(0,1); angles ~ U[-pi, pi]; trap ~ U(0,1).  Q, K, V, Z
    in io_dtype, the rest float32."""
    import math
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    f = dict(device="cuda", dtype=torch.float32, generator=g)
    sN = 1.0 / math.sqrt(N)
    t = dict(Q=(torch.randn(B, L, H, N, **f) * sN).to(io_dtype), K=(torch.randn(B, L, H, N, **f) * sN).to(io_dtype),
             V=torch.randn(B, L, H, P, **f).to(io_dtype), Z=torch.randn(B, L, H, P, **f).to(io_dtype))
    t["DT"] = torch.nn.functional.softplus(torch.randn(B, H, L, **f) * 0.5 - 2.0)
    A = -torch.exp(torch.rand(H, **f) * math.log(16.0))
    t["ADT"] = (A[None, :, None] * t["DT"]).contiguous()
    t["Trap"] = torch.rand(B, H, L, **f)
    t["Angles"] = (torch.rand(B, L, H, R, **f) * 2 - 1) * math.pi
    t["Q_bias"] = torch.randn(H, N, **f) * sN
    t["K_bias"] = torch.randn(H, N, **f) * sN
    t["D"] = torch.randn(H, **f)
    return t


def heads_to_numpy(t, heads):
    """The inputs of a subset of heads as a standalone float32 numpy problem (the scan
    is independent per (batch, head)), for the oracle."""
    import torch
    idx = torch.as_tensor(heads, device="cuda")
    sel = dict(Q=(2, "Q"), K=(2, "K"), V=(2, "V"), Z=(2, "Z"), Angles=(2, "Angles"), ADT=(1, "ADT"),
               DT=(1, "DT"), Trap=(1, "Trap"), Q_bias=(0, "Q_bias"), K_bias=(0, "K_bias"), D=(0, "D"))
    return {k: t[name].index_select(dim, idx).float().cpu().numpy() for k, (dim, name) in sel.items()}


__all__ = ["I", "M", "rel", "oracle_scan", "to_dev", "hip_scan", "ARG_ORDER", "device_scan_inputs",
           "heads_to_numpy"]
