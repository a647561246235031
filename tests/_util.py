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


__all__ = ["I", "M", "rel", "oracle_scan", "to_dev", "hip_scan", "ARG_ORDER"]
