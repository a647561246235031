"""MI355X (gfx950) Mamba3 SISO state-scan operator.

Prefill: ``mamba3_siso_hip`` (the reference's mamba3_siso_triton signature),
``mamba3_ssd_chunked_hip`` (the pure-JAX oracle's signature) and
``mamba3_siso_hip_carry`` (prefill with the recurrent carry in and out) and
``mamba3_ssd_chunked_shared_hip`` (the fused path's contract: B and C shared over
heads, operands in ``pallas_compute_dtype``, the reference's MAMBA3_PALLAS_DTYPE knob).
Backward: ``mamba3_siso_hip`` is differentiable (torch autograd, the reference's
custom_vjp); ``mamba3_siso_hip_bwd`` returns all eleven input gradients directly;
``mamba3_siso_hip_fwd_train`` / ``mamba3_ssd_chunked_shared_hip_fwd_train`` are the
training forwards whose residuals the backward reads.
Decode: ``rnn_step_hip`` (the reference's rnn_step contract, batched).
Layer: ``Mamba3Layer`` (Mamba3SSM's forward: projections, BCNorm, decay, scan,
output norm); ``Mamba3Stack`` (the embedding and SequenceLayer blocks around it).
All run hand-written HIP kernels through the C ABI of include/mamba3_scan.h;
nothing here computes on the CPU.
"""
from ._lib import Mamba3LibraryError, load  # noqa: F401
from .decode import recurrent_angle_mode, recurrent_diagonal_mode, rnn_step_hip  # noqa: F401
from .layer import Mamba3Layer  # noqa: F401
from .stack import Mamba3Stack  # noqa: F401
from .ops import (mamba3_contraction_precision_mode, mamba3_siso_hip, mamba3_siso_hip_bwd,  # noqa: F401
                  mamba3_siso_hip_fwd_train, mamba3_siso_hip_carry, mamba3_ssd_chunked_hip, mamba3_ssd_chunked_shared_hip,
                  mamba3_ssd_chunked_shared_hip_bwd, mamba3_ssd_chunked_shared_hip_fwd_train, new_carry,
                  pallas_compute_dtype)

__all__ = ["mamba3_siso_hip", "mamba3_siso_hip_bwd", "mamba3_siso_hip_fwd_train", "mamba3_ssd_chunked_hip",
           "mamba3_ssd_chunked_shared_hip", "mamba3_ssd_chunked_shared_hip_bwd", "mamba3_siso_hip_carry", "new_carry",
           "rnn_step_hip", "Mamba3Layer", "Mamba3Stack", "recurrent_angle_mode", "recurrent_diagonal_mode", "load",
           "Mamba3LibraryError", "mamba3_contraction_precision_mode", "mamba3_ssd_chunked_shared_hip_fwd_train",
           "pallas_compute_dtype"]
