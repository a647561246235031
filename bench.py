"""Benchmark: Mamba3 chunked scan throughput on one MI355X (+ roofline, CPU baseline).

Headline workload: the bf16 chunked Mamba3 SISO scan
forward at B=8, L=4096, H=32, P=64, N=128, R=32, chunk 64, with fp32 state and
accumulation; synthetic inputs with the configuration's seeded distributions,
generated on the device before timing (inputs resident in HBM).  A "step" is
one scan call over the whole batch (one kernel launch).  ``value`` is tokens/s
over the batch (B*L tokens per step, every head included).

Also reported on the same JSON line:
  roofline      for the scan kernel: algorithmic bytes per launch /
                mean kernel time from HIP events on the launch stream
  cpu_baseline  the numpy float32 restatement of the reference scan
                (oracle/, the reference's own JAX is not installed) timed on
                the host on a bounded sample (one of the 8 sequences)
  secondary     decode state update (config 4, HBM GB/s), the long-context
                scan (config 3, bf16 and float32 I/O), the shared-B/C scan and its backward (recomputing,
                and the training pair), the float32-I/O scan, the scan backward at
                config 2 and at config 3's shape (recomputing its chunk states) and the
                training pair (forward with residuals, backward from them), with bf16
                and with float32 I/O (what the model's training hands the scan),
                each with its own roofline, the scan forward, backward and training
                pair at config 5's layer shape (B=4, L=12288, 24 heads: 96 pairs, the
                sequence split and the split walk), the 12-layer backbone prefill
                with its log-probabilities (config 5), its training step (loss and
                gradients) and its generation step (one token for each of 512 sequences
                through every layer's decode kernel), the mixer layer's training step
                at config 5's layer shape, and, at the shape the reference publishes its
                per-layer training times for (d_model 1024, one 13,000-token
                sequence: docs/training.md:106-112, 283-294), the fused path's scan
                forward + backward and the layer's training step beside those times

Before the warm-up of the headline, the kernel is launched untimed until at least
100 launches and 0.3 s have run (the GPU clocks ramp up over the first ~100
launches of a process); the JSON line reports this as ``clock_settle``, apart from
``warmup``.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--no-secondary]
                       [--mode scan|decode|long|bwd|bwd3|bwd5|train|shared|shared_bwd|layer|layer_train|stack|stack_train|
                               stack_step|copy|fp32]
                       [--io bf16|f32]   (--mode bwd / train)
       python bench.py --mode traffic --pmc-dir DIR   (writes the traffic JSON of
                       the headline kernel from rocprofv3 --pmc FETCH_SIZE /
                       WRITE_SIZE runs of the scan and of the copy kernel)
"""
from __future__ import annotations

import argparse
import glob
import hashlib
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sigma-0_amd"))

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3   # MI355X dense float32 matrix
METRIC = "Mamba3 scan tokens/s + % of MFMA/HBM roofline, bf16 B=8 L=4096 H=32"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "scan_chunked_bf16_config2_traffic.json")
SCAN_KERNEL = "scan_chunked_kernelIDF16bLi64ELi128ELi64ELi32ELi12ELb0E"
# the sources the headline kernel is built from: the traffic measured for one
# version of them says nothing about another
KERNEL_SOURCES = ("sigma-0_amd/csrc/m3_scan_chunked.hip", "sigma-0_amd/csrc/m3_chunk_block.h",
                  "sigma-0_amd/csrc/m3_chunk_common.h", "sigma-0_amd/csrc/m3_common.h", "sigma-0_amd/csrc/m3_scan.h",
                  "sigma-0_amd/build.py")       # the compile flags too


def kernel_sources_sha():
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def scan_bytes(B, L, H, N, P, R, s_io):
    """Algorithmic HBM bytes of one prefill call: every input read once, Out
    written once -- Q, K (N each), V, Z, Out (P each) at s_io bytes, ADT, DT,
    Trap and R angle rates in f32 per token-head (biases negligible)."""
    return B * L * H * ((2 * N + 3 * P) * s_io + 3 * 4 + R * 4)


def scan_flops(B, L, H, N, P, CS):
    """Dense-tile SSD FLOP count per call: 2*CS*N + 2*CS*P + 4*P*N per token-head."""
    return B * L * H * (2 * CS * N + 2 * CS * P + 4 * P * N)


def shared_bytes(B, L, H, N, P, R, s_io):
    """Algorithmic HBM bytes of one call of the fused path's contract: Q, K and the
    angle rates read once per token (shared over heads), V, Z, Out and ADT, DT,
    Trap per token-head."""
    return B * L * (2 * N * s_io + R * 4) + B * L * H * (3 * P * s_io + 3 * 4)


def bwd_bytes(B, L, H, N, P, R, s_io):
    """Algorithmic HBM bytes of one backward call: the forward's inputs and dOut read
    once (Q, K; V, Z, dOut at s_io; ADT, DT, Trap, angles f32), every gradient
    written once (dQ, dK; dV, dZ at s_io; dADT, dDT, dTrap, dAngles f32), per
    token-head.  The chunk states it keeps in its workspace are not counted."""
    return B * L * H * ((2 * N + 3 * P) * s_io + 3 * 4 + R * 4 + (2 * N + 2 * P) * s_io + 3 * 4 + R * 4)


def bwd_flops(B, L, H, N, P, CS, saved_y=False):
    """Dense-tile MFMA FLOP count of one backward call at the kernel's chunk CS (the
    MFMA work the kernel executes: the intra-chunk tiles are counted whole, as in the
    forward's dense-tile formula), per token-head: the chunk's
    S = q~ k~^T, dP = dy v^T, y and dV (intra-chunk S v / S^T dy, inter-chunk q~ h and
    k~ G), the adjoint update dy^T q~, dq~ and dk~ (dP k~ + dy h, dP^T q~ + v G):
    3 (2 CS N) + 3 (2 CS P) + 5 (2 P N).  saved_y: the float32 training pair's
    backward, which reads the output before the gate instead of forming y (one
    2 CS P and one 2 P N term fewer)."""
    if saved_y:
        return B * L * H * (6 * CS * N + 4 * CS * P + 8 * P * N)
    return B * L * H * (6 * CS * N + 6 * CS * P + 10 * P * N)


def decode_bytes(B, H, N, P, R, s_in, s_out):
    """Per decode step: f32 state, angle, k and v carries read and written,
    step inputs (x, z, B, C at s_in; adt, dt, trap, R angles f32) and y."""
    return B * H * (2 * P * N * 4 + 2 * R * 4 + 2 * N * 4 + 2 * P * 4 + (2 * P + 2 * N) * s_in
                    + 3 * 4 + R * 4 + P * s_out)


def make_scan_inputs(torch, B, L, H, N, P, R, seed, io_dtype, device="cuda"):
    """Seeded synthetic scan inputs on the device (config distributions:
    x, z ~ N(0,1); dt = softplus(N(-2,0.5)); A_h = -exp(U[0, ln 16]);
    B, C ~ N(0,1)/sqrt(N); biases ~ N(0,1)/sqrt(N); D ~ N(0,1);
    angles ~ U[-pi, pi]; trap ~ U(0,1))."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    f = dict(device=device, dtype=torch.float32, generator=g)
    sN = 1.0 / math.sqrt(N)
    Q = (torch.randn(B, L, H, N, **f) * sN).to(io_dtype)
    K = (torch.randn(B, L, H, N, **f) * sN).to(io_dtype)
    V = torch.randn(B, L, H, P, **f).to(io_dtype)
    Z = torch.randn(B, L, H, P, **f).to(io_dtype)
    DT = torch.nn.functional.softplus(torch.randn(B, H, L, **f) * 0.5 - 2.0)
    A = -torch.exp(torch.rand(H, **f) * math.log(16.0))
    ADT = (A[None, :, None] * DT).contiguous()
    Trap = torch.rand(B, H, L, **f)
    Ang = (torch.rand(B, L, H, R, **f) * 2 - 1) * math.pi
    Qb = torch.randn(H, N, **f) * sN
    Kb = torch.randn(H, N, **f) * sN
    D = torch.randn(H, **f)
    return (Q, K, V, ADT, DT, Trap, Qb, Kb, Ang, D, Z)


def clock_settle(torch, fn, min_launches=100, min_seconds=0.3):
    """Untimed launches until at least min_launches have run and min_seconds have
    passed: the GPU clocks ramp up under load over about the first 100 launches of
    this kernel in a process, whatever the warm-up count asked for."""
    t0 = time.perf_counter()
    n = 0
    while True:
        for _ in range(10):
            fn()
        n += 10
        torch.cuda.synchronize()
        if n >= min_launches and time.perf_counter() - t0 >= min_seconds:
            return {"launches": n, "seconds": round(time.perf_counter() - t0, 3)}


def time_calls(torch, fn, steps, warmup):
    """Warm up, then time `steps` calls: wall clock between synchronisations and
    per-call HIP events on the current stream (where the kernels launch)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    t0 = time.perf_counter()
    for s, e in ev:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    kern = sum(s.elapsed_time(e) for s, e in ev) / steps / 1e3
    return wall, kern


def bench_scan(torch, B, L, H, N, P, R, CS, steps, warmup, seed, settle=False, io_dtype=None):
    from mamba3_rocm import mamba3_siso_hip
    io_dtype = io_dtype or torch.bfloat16
    args = make_scan_inputs(torch, B, L, H, N, P, R, seed, io_dtype)
    fn = lambda: mamba3_siso_hip(*args, chunk_size=CS)  # noqa: E731
    settled = clock_settle(torch, fn) if settle else None
    wall, kern = time_calls(torch, fn, steps, warmup)
    nbytes = scan_bytes(B, L, H, N, P, R, args[0].element_size())
    return dict(wall_s=wall, kernel_s=kern, bytes=nbytes, flops=scan_flops(B, L, H, N, P, CS),
                flops32=scan_flops(B, L, H, N, P, min(CS, 32)), achieved_gbs=nbytes / kern / 1e9, settle=settled)


def bwd_chunk(torch, io_dtype):
    """The backward kernels' chunk: 64 tokens with bf16 I/O, 32 with float32."""
    return 64 if io_dtype == torch.bfloat16 else 32


def bench_bwd(torch, B, L, H, N, P, R, CS, steps, warmup, seed, io_dtype=None):
    """Backward of the scan (all eleven input gradients) on the config's inputs and a
    N(0, 1) output cotangent."""
    from mamba3_rocm import mamba3_siso_hip_bwd
    io_dtype = io_dtype or torch.bfloat16
    args = make_scan_inputs(torch, B, L, H, N, P, R, seed, io_dtype)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1000)
    dout = torch.randn(B, L, H, P, device="cuda", generator=g).to(io_dtype)
    fn = lambda: mamba3_siso_hip_bwd(*args, dout, chunk_size=CS)  # noqa: E731
    wall, kern = time_calls(torch, fn, steps, warmup)
    nbytes = bwd_bytes(B, L, H, N, P, R, args[0].element_size())
    flops = bwd_flops(B, L, H, N, P, bwd_chunk(torch, io_dtype))
    return dict(wall_s=wall, kernel_s=kern, bytes=nbytes, achieved_gbs=nbytes / kern / 1e9, flops=flops)


def bench_train(torch, B, L, H, N, P, R, CS, steps, warmup, seed, io_dtype=None):
    """The training pair on the config's inputs: the forward that also writes the
    backward's residuals (the state and rope angle entering every chunk and, float32,
    the output before the gate) and the backward that reads them instead of
    recomputing the chunk states and (float32) y -- the
    reference's mamba3_siso_fwd / mamba3_siso_bwd(saved, ...) (mamba3_ops.py:788-902).
    Each is timed on its own (HIP events), with an N(0, 1) output cotangent."""
    from mamba3_rocm import mamba3_siso_hip_bwd, mamba3_siso_hip_fwd_train
    io_dtype = io_dtype or torch.bfloat16
    args = make_scan_inputs(torch, B, L, H, N, P, R, seed, io_dtype)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1000)
    dout = torch.randn(B, L, H, P, device="cuda", generator=g).to(io_dtype)
    _, saved = mamba3_siso_hip_fwd_train(*args, chunk_size=CS)
    fwd = lambda: mamba3_siso_hip_fwd_train(*args, chunk_size=CS)  # noqa: E731
    bwd = lambda: mamba3_siso_hip_bwd(*args, dout, chunk_size=CS, saved=saved)  # noqa: E731
    wf, kf = time_calls(torch, fwd, steps, warmup)
    wb, kb = time_calls(torch, bwd, steps, warmup)
    s_io = args[0].element_size()
    fbytes = scan_bytes(B, L, H, N, P, R, s_io) + saved.numel()       # + the residuals written
    bbytes = bwd_bytes(B, L, H, N, P, R, s_io)
    return dict(fwd_s=kf, bwd_s=kb, wall_s=wf + wb, saved_bytes=saved.numel(),
                fwd_gbs=fbytes / kf / 1e9, bwd_gbs=bbytes / kb / 1e9,
                fwd_flops=scan_flops(B, L, H, N, P, bwd_chunk(torch, io_dtype)),
                bwd_flops=bwd_flops(B, L, H, N, P, bwd_chunk(torch, io_dtype),
                                    saved_y=io_dtype == torch.float32 and args[10] is not None))


def bench_shared(torch, B, L, H, N, P, R, CS, steps, warmup, seed):
    """Config 2 with B, C and the angle rates shared over heads (the fused path)."""
    from mamba3_rocm import mamba3_ssd_chunked_shared_hip
    Q, K, V, ADT, DT, Trap, Qb, Kb, Ang, D, Z = make_scan_inputs(torch, B, L, H, N, P, R, seed, torch.bfloat16)
    Qs, Ks, Angs = Q[:, :, 0].contiguous(), K[:, :, 0].contiguous(), Ang[:, :, 0].contiguous()
    fn = lambda: mamba3_ssd_chunked_shared_hip(Qs, Ks, V, ADT, DT, Trap, Angs, Qb, Kb, D, Z,  # noqa: E731
                                               chunk_size=CS)
    wall, kern = time_calls(torch, fn, steps, warmup)
    nbytes = shared_bytes(B, L, H, N, P, R, 2)
    return dict(wall_s=wall, kernel_s=kern, bytes=nbytes, achieved_gbs=nbytes / kern / 1e9)


def _shared_inputs(torch, B, L, H, N, P, R, seed, io_dtype):
    Q, K, V, ADT, DT, Trap, Qb, Kb, Ang, D, Z = make_scan_inputs(torch, B, L, H, N, P, R, seed, io_dtype)
    return (Q[:, :, 0].contiguous(), K[:, :, 0].contiguous(), V, ADT, DT, Trap, Ang[:, :, 0].contiguous(),
            Qb, Kb, D, Z)


def shared_bwd_bytes(B, L, H, N, P, R, s_io):
    """Algorithmic HBM bytes of one backward call of the fused path's contract: the
    forward's inputs and dOut read once, every gradient written once, with Q, K, the
    angle rates and their gradients once per token (shared over heads)."""
    return (B * L * (2 * N * s_io + R * 4) * 2
            + B * L * H * ((3 * P * s_io + 3 * 4) + (2 * P * s_io + 3 * 4)))


def bench_shared_bwd(torch, B, L, H, N, P, R, CS, steps, warmup, seed):
    """The fused path's backward at config 2 (shared Q, K and angle rates): the
    recomputing backward, and the training pair (forward with residuals, backward
    from them), each timed on its own with an N(0, 1) output cotangent."""
    from mamba3_rocm import mamba3_ssd_chunked_shared_hip_bwd, mamba3_ssd_chunked_shared_hip_fwd_train
    args = _shared_inputs(torch, B, L, H, N, P, R, seed, torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1000)
    dout = torch.randn(B, L, H, P, device="cuda", generator=g).to(torch.bfloat16)
    _, saved = mamba3_ssd_chunked_shared_hip_fwd_train(*args, chunk_size=CS)
    bwd = lambda: mamba3_ssd_chunked_shared_hip_bwd(*args, dout, chunk_size=CS)  # noqa: E731
    fwd_tr = lambda: mamba3_ssd_chunked_shared_hip_fwd_train(*args, chunk_size=CS)  # noqa: E731
    bwd_sv = lambda: mamba3_ssd_chunked_shared_hip_bwd(*args, dout, chunk_size=CS, saved=saved)  # noqa: E731
    wb, kb = time_calls(torch, bwd, steps, warmup)
    wf, kf = time_calls(torch, fwd_tr, steps, warmup)
    ws, ks = time_calls(torch, bwd_sv, steps, warmup)
    nbytes = shared_bwd_bytes(B, L, H, N, P, R, 2)
    return dict(bwd_s=kb, bwd_wall_s=wb, fwd_train_s=kf, bwd_saved_s=ks, pair_wall_s=wf + ws, bytes=nbytes,
                saved_bytes=saved.numel())


def bench_layer(torch, B, L, d_model, steps, warmup, seed):
    """One Mamba3 mixer layer forward (config 5's layer: d_model 768, 24 heads of 64,
    d_state 128, bf16 compute) on a (B, L, d_model) float32 input."""
    from mamba3_rocm import Mamba3Layer
    from mamba3_rocm.layer import init_params
    params = init_params(d_model, seed, "cuda")
    layer = Mamba3Layer(params, d_model, dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    x = torch.randn(B, L, d_model, device="cuda", generator=g)
    wall, kern = time_calls(torch, lambda: layer(x), steps, warmup)
    gemm_flops = 2 * B * L * d_model * (layer.d_in_proj + layer.d_inner)
    return dict(wall_s=wall, kernel_s=kern, gemm_flops=gemm_flops)


def bench_stack(torch, B, L, d_model, n_layers, vocab, steps, warmup, seed):
    """Config 5: the Mamba3 backbone prefill (embedding, n_layers SequenceLayer blocks
    with half_glu1 and prenorm around the mixer, decoder and log_softmax) on token ids
    drawn uniformly from the vocabulary; bf16 compute, random-init parameters."""
    from mamba3_rocm import Mamba3Stack
    from mamba3_rocm.stack import init_params
    params = init_params(vocab, d_model, n_layers, seed, "cuda")
    stack = Mamba3Stack(params, d_model, activation="half_glu1", prenorm=True, dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    ids = torch.randint(0, vocab, (B, L), device="cuda", generator=g)
    wall, kern = time_calls(torch, lambda: stack.logits(ids), steps, warmup)
    layer = stack.blocks[0]["mixer"]
    gemm_flops = 2 * B * L * d_model * (n_layers * (layer.d_in_proj + layer.d_inner + d_model) + vocab)
    return dict(wall_s=wall, kernel_s=kern, gemm_flops=gemm_flops)


def bench_stack_train(torch, B, L, d_model, n_layers, vocab, steps, warmup, seed):
    """Config 5's backbone training step: Mamba3Stack.loss_and_grads (forward with
    the residuals, the mean next-token NLL of random targets, gradients of every
    parameter; no optimizer) on token ids drawn uniformly from the vocabulary."""
    from mamba3_rocm import Mamba3Stack
    from mamba3_rocm.stack import init_params
    params = init_params(vocab, d_model, n_layers, seed, "cuda")
    stack = Mamba3Stack(params, d_model, activation="half_glu1", prenorm=True, dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    ids = torch.randint(0, vocab, (B, L), device="cuda", generator=g)
    tg = torch.randint(0, vocab, (B, L), device="cuda", generator=g)
    wall, kern = time_calls(torch, lambda: stack.loss_and_grads(ids, tg), steps, warmup)
    return dict(wall_s=wall, kernel_s=kern)


def bench_stack_step(torch, B, L0, d_model, n_layers, vocab, steps, warmup, seed):
    """Config 5's backbone generating: a prefill of L0 tokens per sequence (untimed),
    then Mamba3Stack.step, one token for each of the B sequences per step (every
    layer's decode kernel on its carry, the block kernels and the head's
    log-probabilities), issued from the host step by step and replayed as one HIP
    graph (Mamba3Stack.step_graph)."""
    from mamba3_rocm import Mamba3Stack
    from mamba3_rocm.stack import init_params
    params = init_params(vocab, d_model, n_layers, seed, "cuda")
    stack = Mamba3Stack(params, d_model, activation="half_glu1", prenorm=True, dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    ids = torch.randint(0, vocab, (B, L0 + 1), device="cuda", generator=g)
    _, state = stack.prefill(ids[:, :L0])
    tok = ids[:, L0].contiguous()
    wall, kern = time_calls(torch, lambda: stack.step(tok, state), steps, warmup)
    graph = stack.step_graph(state)
    gwall, gkern = time_calls(torch, lambda: graph(tok), steps, warmup)
    return dict(wall_s=wall, kernel_s=kern, graph_wall_s=gwall, graph_kernel_s=gkern)


def bench_layer_train(torch, B, L, d_model, steps, warmup, seed):
    """The mixer layer's training step (24 heads of 64 at config 5's d_model 768, 32 at
    the reference's published d_model 1024): train_forward and the backward to x and
    every parameter (bf16 compute, float32 parameters, no optimizer), and the plain
    forward on its own."""
    from mamba3_rocm import Mamba3Layer
    from mamba3_rocm.layer import init_params
    params = {k: v.requires_grad_(True) for k, v in init_params(d_model, seed, "cuda").items()}
    layer = Mamba3Layer(params, d_model, dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 1)
    x = torch.randn(B, L, d_model, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    dout = torch.randn(B, L, d_model, device="cuda", generator=g).to(torch.bfloat16)

    def step():
        for t in [x, *params.values()]:
            t.grad = None
        layer.train_forward(x).backward(dout)
    wall, kern = time_calls(torch, step, steps, warmup)
    fwd_wall, fwd_kern = time_calls(torch, lambda: layer(x), steps, warmup)
    return dict(wall_s=wall, kernel_s=kern, fwd_s=fwd_kern)


def bench_decode(torch, B, H, N, P, R, steps, warmup, seed):
    """Config 4: `steps` consecutive decode steps in place on a B=512 carry."""
    from mamba3_rocm import rnn_step_hip
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    f = dict(device="cuda", dtype=torch.float32, generator=g)
    sN = 1.0 / math.sqrt(N)
    carry = (torch.rand(B, H, R, **f) * 2 * math.pi, torch.randn(B, H, P, N, **f) * 0.1,
             torch.randn(B, H, N, **f) * sN, torch.randn(B, H, P, **f))
    T = steps + warmup
    bf = torch.bfloat16
    xs = torch.randn(T, B, H, P, **f).to(bf)
    zs = torch.randn(T, B, H, P, **f).to(bf)
    bs = (torch.randn(T, B, H, N, **f) * sN).to(bf)
    cs = (torch.randn(T, B, H, N, **f) * sN).to(bf)
    dts = torch.nn.functional.softplus(torch.randn(T, B, H, **f) * 0.5 - 2.0)
    A = -torch.exp(torch.rand(H, **f) * math.log(16.0))
    adts = A[None, None, :] * dts
    traps = torch.sigmoid(torch.rand(T, B, H, **f))
    angs = (torch.rand(T, B, H, R, **f) * 2 - 1) * math.pi
    Bb, Cb, D = torch.randn(H, N, **f) * sN, torch.randn(H, N, **f) * sN, torch.randn(H, **f)
    step = [0]

    def fn():
        i = step[0]
        step[0] += 1
        rnn_step_hip(carry, (xs[i], zs[i], bs[i], cs[i], adts[i], dts[i], traps[i], angs[i]),
                     Bb, Cb, D, angle_mode="wrapped", diag_mode="current")

    wall, kern = time_calls(torch, fn, steps, warmup)
    nbytes = decode_bytes(B, H, N, P, R, 2, 4)
    return dict(wall_s=wall, kernel_s=kern, bytes=nbytes, achieved_gbs=nbytes / kern / 1e9)


def bench_copy(torch, nbytes, steps, warmup):
    """Plain device copy of a known size: calibration kernel for the PMC
    FETCH_SIZE / WRITE_SIZE counters."""
    n = nbytes // 2
    x = torch.empty(n, dtype=torch.bfloat16, device="cuda").normal_()
    y = torch.empty_like(x)
    wall, kern = time_calls(torch, lambda: y.copy_(x), steps, warmup)
    return dict(kernel_s=kern, read_bytes=n * 2, write_bytes=n * 2,
                achieved_gbs=2 * n * 2 / kern / 1e9)


def cpu_baseline(min_seconds=10.0):
    """Numpy float32 restatement of the reference scan (oracle/mamba3_ref.py,
    following mamba3_jax.py:62-419 with the dense phase-5 state pass) over the
    sequences of the headline workload (4096 tokens x 32 heads each), one at a
    time until at least min_seconds of compute (at most all 8)."""
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import inputs as I
    from oracle import mamba3_ref as M
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    Bfull, L, H, N, P, R, CS = 8, 4096, 32, 128, 64, 32, 64
    spent, nseq = 0.0, 0
    while nseq < Bfull and spent < min_seconds:
        d = I.scan_inputs(1, L, H, N, P, R, seed=2 + nseq, bf16=True)
        args = (d["Q"], d["K"], d["V"], d["ADT"], d["DT"], d["Trap"], d["Angles"], d["Q_bias"],
                d["K_bias"], d["D"], d["Z"])
        t0 = time.perf_counter()
        M.mamba3_ssd_chunked_batched(*args, chunk_size=CS, dtype=np.float32)
        spent += time.perf_counter() - t0
        nseq += 1
        del d, args
    return {"value": round(nseq * L / spent, 1), "unit": "tokens/s", "cores": int(threads),
            "kind": "port",
            "sample": (f"numpy float32 restatement of mamba3_ssd_chunked_jax (reference JAX not "
                       f"installed), {nseq} of the 8 sequences of the headline workload (L=4096, "
                       f"H=32, N=128, P=64, chunk 64), {spent:.1f} s of compute, "
                       f"BLAS threads={threads}, host={len(os.sched_getaffinity(0))} cores"),
            "other": cpu_baseline_other()}


def cpu_baseline_other(decode_seconds=4.0):
    """The other CPU baselines of the measurement plan, on the same host: config 1
    whole (B=2, L=1024, H=8, N=P=64, R=16, chunk 64, float32) through the scan
    restatement, and decode config 4 through the numpy float32 rnn_step restatement
    (mamba3.py:498-562) on 64 of its 512 batch rows, steps until decode_seconds."""
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import inputs as I
    from oracle import mamba3_ref as M
    d = I.scan_inputs(2, 1024, 8, 64, 64, 16, seed=1)
    t0 = time.perf_counter()
    M.mamba3_ssd_chunked_batched(d["Q"], d["K"], d["V"], d["ADT"], d["DT"], d["Trap"], d["Angles"],
                                 d["Q_bias"], d["K_bias"], d["D"], d["Z"], chunk_size=64, dtype=np.float32)
    c1 = time.perf_counter() - t0
    rows, max_steps = 64, 256
    e = I.decode_inputs(rows, 32, 128, 64, 32, 32, seed=4)
    carry = (e["theta"], e["h"], e["k_prev"], e["v_prev"])
    spent, steps = 0.0, 0
    while steps < max_steps and spent < decode_seconds:
        t = steps % 32
        step_in = tuple(e[k][t] for k in ("x", "z", "Bt", "Ct", "adt", "dt", "trap", "ang"))
        t0 = time.perf_counter()
        carry, _ = M.rnn_step(carry, step_in, e["B_bias"], e["C_bias"], e["D"], dtype=np.float32)
        spent += time.perf_counter() - t0
        steps += 1
    return {"config1_scan": {"value": round(2 * 1024 / c1, 1), "unit": "tokens/s",
                             "sample": f"config 1 whole (2 x 1024 tokens, 8 heads), {c1:.2f} s"},
            "decode_config4": {"value": round(rows * steps / spent, 1), "unit": "tokens/s",
                               "sample": (f"{rows} of the 512 batch rows, {steps} steps of rnn_step "
                                          f"(32 heads, N=128, P=64), {spent:.1f} s")}}


def load_traffic():
    """HBM bytes per launch of the headline kernel from the committed PMC measurement,
    or None when that measurement was taken on other kernel sources (stale) or is
    missing."""
    try:
        with open(TRAFFIC_FILE) as fh:
            d = json.load(fh)
    except (OSError, ValueError):
        return None, "missing"
    if d.get("kernel_sources_sha") != kernel_sources_sha():
        return None, "stale: measured on other kernel sources"
    return d.get("traffic_bytes"), os.path.relpath(TRAFFIC_FILE, ROOT)


def pmc_per_dispatch(run_dir, kernel_substr, counter):
    """Mean of `counter` (rocprofv3 --pmc CSV, KiB per dispatch) over the dispatches of
    the kernels whose name contains kernel_substr."""
    vals = []
    for path in glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"), recursive=True):
        import csv
        with open(path, newline="") as fh:
            for row in csv.DictReader(fh):
                if row["Counter_Name"] == counter and kernel_substr in row["Kernel_Name"]:
                    vals.append(float(row["Counter_Value"]))
    if not vals:
        raise SystemExit(f"no {counter} rows for {kernel_substr!r} under {run_dir}")
    return sum(vals) / len(vals), len(vals)


def write_traffic(pmc_dir, kernel_avg_us=None):
    """Traffic JSON of the headline kernel from four rocprofv3 --pmc runs under
    pmc_dir: scan_FETCH_SIZE, scan_WRITE_SIZE (bench.py --steps 3 --warmup 1
    --no-cpu-baseline --no-secondary) and copy_FETCH_SIZE, copy_WRITE_SIZE (bench.py
    --mode copy: a 1 GiB device copy that reads and writes 2^30 bytes), which give the
    counters' scale factors on this part."""
    copy_kernel = "copyBuffer"
    cf, _ = pmc_per_dispatch(os.path.join(pmc_dir, "copy_FETCH_SIZE"), copy_kernel, "FETCH_SIZE")
    cw, _ = pmc_per_dispatch(os.path.join(pmc_dir, "copy_WRITE_SIZE"), copy_kernel, "WRITE_SIZE")
    ff, fw = (1 << 30) / (cf * 1024), (1 << 30) / (cw * 1024)
    sf, nf = pmc_per_dispatch(os.path.join(pmc_dir, "scan_FETCH_SIZE"), SCAN_KERNEL, "FETCH_SIZE")
    sw, nw = pmc_per_dispatch(os.path.join(pmc_dir, "scan_WRITE_SIZE"), SCAN_KERNEL, "WRITE_SIZE")
    traffic = sf * 1024 * ff + sw * 1024 * fw
    alg = scan_bytes(8, 4096, 32, 128, 64, 32, 2)
    d = {"workload": "mamba3 chunked scan forward, config 2", "kernel": SCAN_KERNEL,
         "kernel_sources_sha": kernel_sources_sha(), "fetch_kib": round(sf, 1), "write_kib": round(sw, 1),
         "dispatches": [nf, nw], "fetch_factor": ff, "write_factor": fw,
         "traffic_bytes": int(round(traffic)), "algorithmic_bytes": alg,
         "traffic_over_algorithmic": round(traffic / alg, 4)}
    if kernel_avg_us:
        d["kernel_avg_us"] = kernel_avg_us
    with open(TRAFFIC_FILE, "w") as fh:
        json.dump(d, fh, indent=1)
    print(json.dumps(d), flush=True)


FLOP_COUNT_NOTE = ("dense-tile MFMA FLOPs at the kernel's own chunk (32 tokens for float32 I/O): the "
                   "matrix work the kernel executes, intra-chunk tiles counted whole")


def bwd_line(r, fp32=False, tokens=8 * 4096):
    """The JSON fields of a backward measurement: time, tokens/s, and its roofline --
    HBM for bf16 I/O; float32 MFMA for float32 I/O, whose dense-tile MFMA work takes
    longer at the float32 peak than its bytes at the HBM peak."""
    d = {"ms": round(r["kernel_s"] * 1e3, 4), "tokens_per_s": round(tokens / r["wall_s"], 1),
         "achieved_gbs": round(r["achieved_gbs"], 1), "frac_hbm": round(r["achieved_gbs"] / HBM_PEAK_GBS, 4)}
    if fp32:
        tf = r["flops"] / r["kernel_s"] / 1e12
        d.update(bound="mfma_fp32", tflops=round(tf, 1), frac_mfma_fp32=round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
                 flop_count=FLOP_COUNT_NOTE)
    return d


def fp32_fwd_line(r):
    """The float32-I/O forward's fields: its dense-tile FLOPs at the kernel's 32-token
    chunk against the float32 MFMA peak, its bytes against HBM, and the fraction of
    whichever roof binds (the longer of the two roofline times)."""
    t_mfma = r["flops32"] / (FP32_MFMA_PEAK_TFLOPS * 1e12)
    t_hbm = r["bytes"] / (HBM_PEAK_GBS * 1e9)
    bound = "mfma_fp32" if t_mfma >= t_hbm else "hbm"
    tf = r["flops32"] / r["kernel_s"] / 1e12
    return {"kernel_ms": round(r["kernel_s"] * 1e3, 4), "bound": bound,
            "roofline_us": round(max(t_mfma, t_hbm) * 1e6, 1), "frac": round(max(t_mfma, t_hbm) / r["kernel_s"], 4),
            "tflops": round(tf, 1), "frac_mfma_fp32": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
            "achieved_gbs": round(r["achieved_gbs"], 1), "frac_hbm": round(r["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "flop_count": FLOP_COUNT_NOTE}


def train_line(r, fp32=False, tokens=8 * 4096):
    """The JSON fields of a training-pair measurement (forward with residuals, backward
    from them); the backward's roofline as in bwd_line."""
    d = {"fwd_with_residuals_ms": round(r["fwd_s"] * 1e3, 4), "bwd_from_residuals_ms": round(r["bwd_s"] * 1e3, 4),
         "step_ms": round((r["fwd_s"] + r["bwd_s"]) * 1e3, 4), "tokens_per_s": round(tokens / r["wall_s"], 1),
         "residual_bytes": r["saved_bytes"], "bwd_achieved_gbs": round(r["bwd_gbs"], 1),
         "bwd_frac_hbm": round(r["bwd_gbs"] / HBM_PEAK_GBS, 4)}
    if fp32:
        tf = r["bwd_flops"] / r["bwd_s"] / 1e12
        d.update(bwd_bound="mfma_fp32", bwd_tflops=round(tf, 1), bwd_frac_mfma_fp32=round(tf / FP32_MFMA_PEAK_TFLOPS, 4))
    return d


def shared_bwd_line(r):
    """The fused path's backward fields: the recomputing backward and the training pair,
    against the contract's algorithmic bytes (shared rows once per token)."""
    return {"ms": round(r["bwd_s"] * 1e3, 4), "tokens_per_s": round(8 * 4096 / r["bwd_wall_s"], 1),
            "achieved_gbs": round(r["bytes"] / r["bwd_s"] / 1e9, 1),
            "frac_hbm": round(r["bytes"] / r["bwd_s"] / 1e9 / HBM_PEAK_GBS, 4),
            "fwd_with_residuals_ms": round(r["fwd_train_s"] * 1e3, 4),
            "bwd_from_residuals_ms": round(r["bwd_saved_s"] * 1e3, 4),
            "pair_step_ms": round((r["fwd_train_s"] + r["bwd_saved_s"]) * 1e3, 4),
            "pair_tokens_per_s": round(8 * 4096 / r["pair_wall_s"], 1),
            "bwd_from_residuals_frac_hbm": round(r["bytes"] / r["bwd_saved_s"] / 1e9 / HBM_PEAK_GBS, 4),
            "residual_bytes": r["saved_bytes"], "algorithmic_bytes": r["bytes"]}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--mode", choices=("scan", "decode", "long", "bwd", "bwd3", "bwd5", "train", "shared", "shared_bwd",
                                       "layer", "layer_train",
                                       "stack", "stack_train", "stack_step", "copy", "fp32", "traffic"),
                    default="scan")
    ap.add_argument("--pmc-dir", default=None, help="--mode traffic: the folder holding the rocprofv3 --pmc runs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--io", choices=("bf16", "f32"), default="bf16", help="--mode bwd / train / long: the I/O dtype")
    args = ap.parse_args()

    if args.mode == "traffic":
        if not args.pmc_dir:
            ap.error("--mode traffic needs --pmc-dir")
        write_traffic(args.pmc_dir)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}): "
              "this build runs the scan on a single MI355X; the batch and head axes shard "
              "across GPUs with no exchange.", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)

    if args.mode == "copy":
        r = bench_copy(torch, 1 << 30, args.steps, args.warmup)
        print(json.dumps({"mode": "copy", **r}), flush=True)
        return
    if args.mode == "decode":
        r = bench_decode(torch, 512, 32, 128, 64, 32, args.steps, args.warmup, seed=4)
        print(json.dumps({"mode": "decode", **r}), flush=True)
        return

    io = torch.float32 if args.io == "f32" else torch.bfloat16
    if args.mode == "bwd":
        # backward at config 2 alone, for profiling
        r = bench_bwd(torch, 8, 4096, 32, 128, 64, 32, 64, args.steps, args.warmup, seed=2, io_dtype=io)
        print(json.dumps({"mode": "bwd", "io_dtype": args.io, **bwd_line(r)}), flush=True)
        return
    if args.mode == "bwd3":
        # the backward and the training pair at config 3's shape (B*H = 32: the split walk)
        r = bench_bwd(torch, 1, 32768, 32, 128, 64, 32, 128, args.steps, args.warmup, seed=3, io_dtype=io)
        t = bench_train(torch, 1, 32768, 32, 128, 64, 32, 128, args.steps, args.warmup, seed=3, io_dtype=io)
        print(json.dumps({"mode": "bwd3", "io_dtype": args.io, **bwd_line(r, tokens=32768),
                          "training_pair": train_line(t, tokens=32768)}), flush=True)
        return
    if args.mode == "bwd5":
        # the scan forward, backward and training pair at config 5's layer shape (B*H = 96:
        # the sequence split and the split walk)
        f = bench_scan(torch, 4, 12288, 24, 128, 64, 32, 64, args.steps, args.warmup, seed=5, io_dtype=io)
        r = bench_bwd(torch, 4, 12288, 24, 128, 64, 32, 64, args.steps, args.warmup, seed=5, io_dtype=io)
        t = bench_train(torch, 4, 12288, 24, 128, 64, 32, 64, args.steps, args.warmup, seed=5, io_dtype=io)
        print(json.dumps({"mode": "bwd5", "io_dtype": args.io, "scan_kernel_ms": round(f["kernel_s"] * 1e3, 4),
                          "scan_frac_hbm": round(f["achieved_gbs"] / HBM_PEAK_GBS, 4),
                          **bwd_line(r, tokens=4 * 12288), "training_pair": train_line(t, tokens=4 * 12288)}),
              flush=True)
        return
    if args.mode == "train":
        # the training pair at config 2 (forward with residuals, backward from them)
        r = bench_train(torch, 8, 4096, 32, 128, 64, 32, 64, args.steps, args.warmup, seed=2, io_dtype=io)
        print(json.dumps({"mode": "train", "io_dtype": args.io, **train_line(r)}), flush=True)
        return
    if args.mode == "layer":
        r = bench_layer(torch, 4, 12288, 768, args.steps, args.warmup, seed=5)
        print(json.dumps({"mode": "layer", "ms": round(r["kernel_s"] * 1e3, 4),
                          "tokens_per_s": round(4 * 12288 / r["wall_s"], 1),
                          "gemm_tflop": round(r["gemm_flops"] / 1e12, 4)}), flush=True)
        return
    if args.mode == "layer_train":
        r = bench_layer_train(torch, 4, 12288, 768, args.steps, args.warmup, seed=5)
        print(json.dumps({"mode": "layer_train", "step_ms": round(r["kernel_s"] * 1e3, 4),
                          "fwd_ms": round(r["fwd_s"] * 1e3, 4),
                          "tokens_per_s": round(4 * 12288 / r["wall_s"], 1)}), flush=True)
        return
    if args.mode == "stack_step":
        r = bench_stack_step(torch, 512, 64, 768, 12, 2112, args.steps, args.warmup, seed=5)
        print(json.dumps({"mode": "stack_step", "B": 512, "ms_per_step": round(r["kernel_s"] * 1e3, 4),
                          "tokens_per_s": round(512 / r["wall_s"], 1),
                          "graph_ms_per_step": round(r["graph_kernel_s"] * 1e3, 4),
                          "graph_tokens_per_s": round(512 / r["graph_wall_s"], 1)}), flush=True)
        return
    if args.mode == "stack_train":
        r = bench_stack_train(torch, 4, 12288, 768, 12, 2112, args.steps, args.warmup, seed=5)
        print(json.dumps({"mode": "stack_train", "step_ms": round(r["kernel_s"] * 1e3, 4),
                          "tokens_per_s": round(4 * 12288 / r["wall_s"], 1)}), flush=True)
        return
    if args.mode == "stack":
        r = bench_stack(torch, 4, 12288, 768, 12, 2112, args.steps, args.warmup, seed=5)
        print(json.dumps({"mode": "stack", "ms": round(r["kernel_s"] * 1e3, 4),
                          "tokens_per_s": round(4 * 12288 / r["wall_s"], 1),
                          "gemm_tflop": round(r["gemm_flops"] / 1e12, 4)}), flush=True)
        return
    if args.mode == "shared":
        r = bench_shared(torch, 8, 4096, 32, 128, 64, 32, 64, args.steps, args.warmup, seed=2)
        print(json.dumps({"mode": "shared", "kernel_ms": round(r["kernel_s"] * 1e3, 4),
                          "tokens_per_s": round(8 * 4096 / r["wall_s"], 1),
                          "achieved_gbs": round(r["achieved_gbs"], 1),
                          "frac_hbm": round(r["achieved_gbs"] / HBM_PEAK_GBS, 4)}), flush=True)
        return
    if args.mode == "fp32":
        # config 2's shape with float32 I/O (what the model hands the scan), for profiling
        r = bench_scan(torch, 8, 4096, 32, 128, 64, 32, 64, args.steps, args.warmup, seed=2,
                       io_dtype=torch.float32)
        print(json.dumps({"mode": "fp32", "tokens_per_s": round(8 * 4096 / r["wall_s"], 1), **fp32_fwd_line(r)}),
              flush=True)
        return
    if args.mode == "shared_bwd":
        r = bench_shared_bwd(torch, 8, 4096, 32, 128, 64, 32, 64, args.steps, args.warmup, seed=2)
        print(json.dumps({"mode": "shared_bwd", **shared_bwd_line(r)}), flush=True)
        return
    if args.mode == "long":
        # config 3 alone (B*H = 32: the sequence split runs), for profiling
        r = bench_scan(torch, 1, 32768, 32, 128, 64, 32, 128, args.steps, args.warmup, seed=3, io_dtype=io)
        if io == torch.float32:
            print(json.dumps({"mode": "long", "io_dtype": "f32", "tokens_per_s": round(32768 / r["wall_s"], 1),
                              **fp32_fwd_line(r)}), flush=True)
            return
        print(json.dumps({"mode": "long", "kernel_ms": round(r["kernel_s"] * 1e3, 4),
                          "tokens_per_s": round(32768 / r["wall_s"], 1),
                          "achieved_gbs": round(r["achieved_gbs"], 1),
                          "frac_hbm": round(r["achieved_gbs"] / HBM_PEAK_GBS, 4)}), flush=True)
        return

    B, L, H, N, P, R, CS = 8, 4096, 32, 128, 64, 32, 64
    r = bench_scan(torch, B, L, H, N, P, R, CS, args.steps, args.warmup, seed=2, settle=True)
    ms = r["wall_s"] * 1e3
    traffic, traffic_src = load_traffic()
    out = {
        "metric": METRIC,
        "value": round(B * L / r["wall_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, config distributions, generated on device)",
        "config": {"workload": "mamba3 chunked scan forward, config 2", "B": B, "L": L, "H": H,
                   "P": P, "N": N, "R": R, "chunk": CS, "io_dtype": "bf16",
                   "state_dtype": "f32"},
        "clock_settle": dict(r["settle"], note="untimed launches of the headline kernel before the "
                             "warm-up, until >= 100 launches and >= 0.3 s (GPU clock ramp)"),
        "roofline": {"bound": "hbm", "achieved": round(r["achieved_gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(r["achieved_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_src, "algorithmic_bytes": r["bytes"],
                     "kernel_ms": round(r["kernel_s"] * 1e3, 4),
                     "mfma_tflops": round(r["flops"] / r["kernel_s"] / 1e12, 1)},
    }
    if not args.no_secondary:
        dec = bench_decode(torch, 512, 32, 128, 64, 32, 256, 16, seed=4)
        lc = bench_scan(torch, 1, 32768, 32, 128, 64, 32, 128, max(5, args.steps // 5), 3, seed=3)
        lc32 = bench_scan(torch, 1, 32768, 32, 128, 64, 32, 128, max(5, args.steps // 5), 3, seed=3,
                          io_dtype=torch.float32)
        bw = bench_bwd(torch, 8, 4096, 32, 128, 64, 32, 64, max(5, args.steps // 5), 3, seed=2)
        tr = bench_train(torch, 8, 4096, 32, 128, 64, 32, 64, max(5, args.steps // 5), 3, seed=2)
        bw32 = bench_bwd(torch, 8, 4096, 32, 128, 64, 32, 64, max(5, args.steps // 10), 2, seed=2,
                         io_dtype=torch.float32)
        tr32 = bench_train(torch, 8, 4096, 32, 128, 64, 32, 64, max(5, args.steps // 10), 2, seed=2,
                           io_dtype=torch.float32)
        sh = bench_shared(torch, 8, 4096, 32, 128, 64, 32, 64, max(5, args.steps // 5), 3, seed=2)
        shb = bench_shared_bwd(torch, 8, 4096, 32, 128, 64, 32, 64, max(5, args.steps // 5), 3, seed=2)
        bw3 = bench_bwd(torch, 1, 32768, 32, 128, 64, 32, 128, max(5, args.steps // 10), 2, seed=3)
        tr3 = bench_train(torch, 1, 32768, 32, 128, 64, 32, 128, max(5, args.steps // 10), 2, seed=3)
        sc5 = bench_scan(torch, 4, 12288, 24, 128, 64, 32, 64, max(5, args.steps // 5), 3, seed=5)
        bw5 = bench_bwd(torch, 4, 12288, 24, 128, 64, 32, 64, max(5, args.steps // 10), 2, seed=5)
        tr5 = bench_train(torch, 4, 12288, 24, 128, 64, 32, 64, max(5, args.steps // 10), 2, seed=5)
        f32 = bench_scan(torch, 8, 4096, 32, 128, 64, 32, 64, max(5, args.steps // 5), 3, seed=2,
                         io_dtype=torch.float32)
        bb = bench_stack(torch, 4, 12288, 768, 12, 2112, 5, 2, seed=5)
        lt5 = bench_layer_train(torch, 4, 12288, 768, max(5, args.steps // 10), 2, seed=5)
        st5 = bench_stack_train(torch, 4, 12288, 768, 12, 2112, 3, 1, seed=5)
        sd5 = bench_stack_step(torch, 512, 64, 768, 12, 2112, 20, 5, seed=5)
        rs = bench_shared_bwd(torch, 1, 13000, 32, 128, 64, 32, 64, max(5, args.steps // 5), 3, seed=6)
        rl = bench_layer_train(torch, 1, 13000, 1024, max(5, args.steps // 5), 3, seed=6)
        out["secondary"] = {
            "decode_config4": {"B": 512, "H": 32, "P": 64, "N": 128, "steps": 256,
                               "us_per_step": round(dec["kernel_s"] * 1e6, 2),
                               "tokens_per_s": round(512 / dec["wall_s"], 1),
                               "achieved_gbs": round(dec["achieved_gbs"], 1),
                               "frac_hbm": round(dec["achieved_gbs"] / HBM_PEAK_GBS, 4)},
            "long_context_config3": {"B": 1, "L": 32768, "H": 32, "chunk": 128,
                                     "kernel_ms": round(lc["kernel_s"] * 1e3, 4),
                                     "tokens_per_s": round(32768 / lc["wall_s"], 1),
                                     "achieved_gbs": round(lc["achieved_gbs"], 1),
                                     "frac_hbm": round(lc["achieved_gbs"] / HBM_PEAK_GBS, 4)},
            "long_context_fp32_io_config3": {"B": 1, "L": 32768, "H": 32, "chunk": 128, "io_dtype": "f32",
                                             "tokens_per_s": round(32768 / lc32["wall_s"], 1), **fp32_fwd_line(lc32)},
            "shared_bc_config2": {"B": 8, "L": 4096, "H": 32, "chunk": 64,
                                  "kernel_ms": round(sh["kernel_s"] * 1e3, 4),
                                  "tokens_per_s": round(8 * 4096 / sh["wall_s"], 1),
                                  "achieved_gbs": round(sh["achieved_gbs"], 1),
                                  "frac_hbm": round(sh["achieved_gbs"] / HBM_PEAK_GBS, 4)},
            "shared_bc_backward_config2": {"B": 8, "L": 4096, "H": 32, "chunk": 64, **shared_bwd_line(shb)},
            "fp32_io_config2": {"B": 8, "L": 4096, "H": 32, "chunk": 64, "io_dtype": "f32",
                                "tokens_per_s": round(8 * 4096 / f32["wall_s"], 1), **fp32_fwd_line(f32)},
            "backward_config2": {"B": 8, "L": 4096, "H": 32, "chunk": 64, **bwd_line(bw)},
            "backward_config3_shape": {"B": 1, "L": 32768, "H": 32, "chunk": 128,
                                       **bwd_line(bw3, tokens=32768)},
            "training_pair_config3_shape": {"B": 1, "L": 32768, "H": 32, "chunk": 128,
                                            **train_line(tr3, tokens=32768)},
            "training_pair_config2": {"B": 8, "L": 4096, "H": 32, "chunk": 64, **train_line(tr)},
            "scan_config5_layer_shape": {"B": 4, "L": 12288, "H": 24, "chunk": 64,
                                         "kernel_ms": round(sc5["kernel_s"] * 1e3, 4),
                                         "tokens_per_s": round(4 * 12288 / sc5["wall_s"], 1),
                                         "achieved_gbs": round(sc5["achieved_gbs"], 1),
                                         "frac_hbm": round(sc5["achieved_gbs"] / HBM_PEAK_GBS, 4)},
            "backward_config5_layer_shape": {"B": 4, "L": 12288, "H": 24, "chunk": 64,
                                             **bwd_line(bw5, tokens=4 * 12288)},
            "training_pair_config5_layer_shape": {"B": 4, "L": 12288, "H": 24, "chunk": 64,
                                                  **train_line(tr5, tokens=4 * 12288)},
            "backward_fp32_io_config2": {"B": 8, "L": 4096, "H": 32, "chunk": 64, "io_dtype": "f32",
                                         **bwd_line(bw32, fp32=True)},
            "training_pair_fp32_io_config2": {"B": 8, "L": 4096, "H": 32, "chunk": 64, "io_dtype": "f32",
                                              **train_line(tr32, fp32=True)},
            "backbone_prefill_config5": {"B": 4, "L": 12288, "layers": 12, "d_model": 768, "vocab": 2112,
                                         "activation": "half_glu1", "prenorm": True, "dtype": "bf16",
                                         "ms": round(bb["kernel_s"] * 1e3, 4),
                                         "tokens_per_s": round(4 * 12288 / bb["wall_s"], 1),
                                         "gemm_tflops": round(bb["gemm_flops"] / bb["kernel_s"] / 1e12, 1)},
            "backbone_train_config5": {"B": 4, "L": 12288, "layers": 12, "d_model": 768, "vocab": 2112,
                                       "activation": "half_glu1", "prenorm": True, "dtype": "bf16",
                                       "loss": "mean next-token NLL, random targets; no optimizer",
                                       "step_ms": round(st5["kernel_s"] * 1e3, 4),
                                       "tokens_per_s": round(4 * 12288 / st5["wall_s"], 1)},
            "backbone_decode_config5": {"B": 512, "prefill": 64, "layers": 12, "d_model": 768, "vocab": 2112,
                                        "dtype": "bf16", "ms_per_step": round(sd5["kernel_s"] * 1e3, 4),
                                        "tokens_per_s": round(512 / sd5["wall_s"], 1),
                                        "graph_ms_per_step": round(sd5["graph_kernel_s"] * 1e3, 4),
                                        "graph_tokens_per_s": round(512 / sd5["graph_wall_s"], 1)},
            "layer_train_config5": {"B": 4, "L": 12288, "d_model": 768, "H": 24, "dtype": "bf16",
                                    "step_ms": round(lt5["kernel_s"] * 1e3, 4),
                                    "fwd_ms": round(lt5["fwd_s"] * 1e3, 4),
                                    "tokens_per_s": round(4 * 12288 / lt5["wall_s"], 1)},
            "reference_layer_shape": {
                "B": 1, "L": 13000, "d_model": 1024, "H": 32, "chunk": 64, "dtype": "bf16",
                "ssd_fwd_bwd_ms": round((rs["fwd_train_s"] + rs["bwd_saved_s"]) * 1e3, 4),
                "ssd_fwd_train_ms": round(rs["fwd_train_s"] * 1e3, 4),
                "ssd_bwd_saved_ms": round(rs["bwd_saved_s"] * 1e3, 4),
                "layer_step_ms": round(rl["kernel_s"] * 1e3, 4),
                "layer_fwd_ms": round(rl["fwd_s"] * 1e3, 4),
                "published_gh200": {"ssd_fwd_bwd_ms": 6.6, "ssd_fwd_ms": 1.7, "layer_step_ms": 13.0,
                                    "source": "docs/training.md:283,291",
                                    "note": "one GH200; its layer step includes the optimizer's share"}},
        }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
