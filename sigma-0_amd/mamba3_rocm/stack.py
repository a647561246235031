"""The Mamba3 backbone around the mixer on gfx950: StackedEncoderModel
(src/base_model/models/seq_model.py:47-118, use_embed_layer=True) of
SequenceLayer blocks (layers.py:108-160) with the Mamba3 mixer (Mamba3Layer).

A block is skip = x; LayerNorm if prenorm; mixer; activation (gelu, full_glu,
half_glu1, half_glu2, with the block's out1/out2 Dense layers in the compute
dtype); x = skip + x; LayerNorm if postnorm.  flax defaults: LayerNorm eps 1e-6,
gelu with the tanh approximation.  The mixer and the block's elementwise work run
the hand-written kernels: m3_block_norm (LayerNorm from the float32 residual
straight to the mixer's dtype, for the first block), m3_block_gelu (the Dense
layers' input) and m3_block_act_norm (the gate, the residual add and the next
block's LayerNorm in one pass; postnorm: this block's).  The Dense layers are
library GEMMs; the embedding lookup is torch's gather.
``logits`` adds the LOB models' per-token head (mode "none"): the decoder Dense
on the float32 features (a library GEMM), then log_softmax in float32 with
m3_log_softmax (lob_seq_model.py:530-542).  Dropout is the identity.
``loss_and_grads`` is a training step's loss and gradients (prenorm stacks): the
mean negative log-likelihood of target tokens under that head, and the gradient of
every parameter as autodiff of the same model gives it.  The backward runs the
hand-written kernels too: m3_log_softmax_nll (the head), m3_block_act_bwd and
m3_block_gelu_bwd (the activation epilogue around the Dense layers' gradients,
library GEMMs), the mixer's backward (Mamba3Layer) and m3_block_norm_bwd (the
prenorm LayerNorm into the residual stream's gradient); the embedding's gradient is
torch's index_add (its float32 sums over repeated tokens are not in a fixed order).
``step_graph`` captures the generation step in a HIP graph.
In a bf16 stack the head's float32 products (the decoder Dense, and in the training
step its two gradients) run as three bf16 products with float32 accumulation:
a b = a_hi b_hi + a_hi b_lo + a_lo b_hi with hi = bf16(a), lo = bf16(a - hi) (split by
m3_split_bf16x3), relative error about 1e-5.  gfx950's matrix cores have no TF32-like
float32 mode and run bf16 at 16 times their float32 rate.  A float32 stack keeps
float32 products.
"""
from __future__ import annotations

from typing import Dict, List

import torch
import torch.nn.functional as F

from . import _lib
from .layer import PARAM_NAMES, Mamba3Layer
from .ops import _IO, _ptr, _stream

ACTIVATIONS = ("gelu", "full_glu", "half_glu1", "half_glu2")
_ACT = dict(gelu=_lib.M3_ACT_GELU, full_glu=_lib.M3_ACT_FULL_GLU, half_glu1=_lib.M3_ACT_HALF_GLU1,
            half_glu2=_lib.M3_ACT_HALF_GLU2)


class Mamba3Stack:
    """Token ids (B, L) -> features (B, L, d_model), float32 residual stream."""

    def __init__(self, params: Dict, d_model: int, activation: str = "half_glu1", prenorm: bool = True,
                 d_state: int = 128, headdim: int = 64, chunk_size: int = 64, dtype: torch.dtype = torch.bfloat16):
        if activation not in ACTIVATIONS:
            raise ValueError(f"activation must be one of {ACTIVATIONS}, got {activation!r}")
        self.activation, self.prenorm, self.dtype, self.d_model = activation, prenorm, dtype, d_model
        self.embed = params["embed"].to(torch.float32).contiguous()
        self.blocks: List[Dict] = []
        for lp in params["layers"]:
            b = dict(mixer=Mamba3Layer(lp["mixer"], d_model, d_state=d_state, headdim=headdim,
                                       chunk_size=chunk_size, dtype=dtype),
                     ln_scale=lp["ln_scale"].float().contiguous(), ln_bias=lp["ln_bias"].float().contiguous())
            for n in ("out1", "out2"):
                b[n + "_w"] = lp[n + "_w"].to(dtype).t().contiguous()     # flax (in, out) -> F.linear (out, in)
                b[n + "_b"] = lp[n + "_b"].to(dtype)
            self.blocks.append(b)
        self.decoder_w = self.decoder_b = None
        self._dec_w3 = self._dec_w3b = None
        if "decoder_w" in params:
            self.decoder_w = params["decoder_w"].float().t().contiguous()
            self.decoder_b = params["decoder_b"].float().contiguous()
            if dtype == torch.bfloat16:
                # split-bf16 operands of the decoder weight (V, D): [hi | lo | hi] along D
                # against the features' [hi | hi | lo], and the same stacked along V
                # against the logits' gradient
                wh = self.decoder_w.to(torch.bfloat16)
                wl = (self.decoder_w - wh.float()).to(torch.bfloat16)
                self._dec_w3 = torch.cat([wh, wl, wh], 1).contiguous()
                self._dec_w3b = torch.cat([wh, wl, wh], 0).contiguous()

    def _block(self, b, x, xin, nxt, mixer=None):
        """SequenceLayer.__call__ (layers.py:108-160) on the float32 residual x (B, L, D).
        Prenorm: xin is this block's normalised input, made by the previous block's
        epilogue (or by m3_block_norm for the first block), and the epilogue makes the
        next block's (nxt) the same way.  ``mixer`` replaces the mixer's forward (the
        prefill and the decode step).  Returns (residual, next block's input)."""
        lib, io, st = _lib.load(), _IO[self.dtype], _stream(x)
        Bn, L, D = x.shape
        mixer = mixer or b["mixer"]
        y = mixer(xin if self.prenorm else x).contiguous()         # compute dtype
        h1 = h2 = None
        if self.activation != "gelu":
            g = torch.empty_like(y)
            _lib.check(lib.m3_block_gelu(_ptr(y), _ptr(g), Bn, L, D, io, st), "m3_block_gelu")
            h2 = F.linear(g, b["out2_w"], b["out2_b"])
            if self.activation == "full_glu":
                h1 = F.linear(g, b["out1_w"], b["out1_b"])
        act = _ACT[self.activation]
        out = torch.empty_like(x)
        if self.prenorm and nxt is None:
            _lib.check(lib.m3_block_act(_ptr(y), _ptr(h1), _ptr(h2), _ptr(x), _ptr(out), Bn, L, D, act, io, st),
                       "m3_block_act")
            return out, None
        if self.prenorm:         # residual and the next block's LayerNorm in one pass
            xn = torch.empty(Bn, L, D, device=x.device, dtype=self.dtype)
            _lib.check(lib.m3_block_act_norm(_ptr(y), _ptr(h1), _ptr(h2), _ptr(x), _ptr(out), _ptr(nxt["ln_scale"]),
                                             _ptr(nxt["ln_bias"]), _ptr(xn), Bn, L, D, 1e-6, act, io, io, st),
                       "m3_block_act_norm")
            return out, xn
        # postnorm: the LayerNorm of skip + act is the residual itself
        _lib.check(lib.m3_block_act_norm(_ptr(y), _ptr(h1), _ptr(h2), _ptr(x), None, _ptr(b["ln_scale"]),
                                         _ptr(b["ln_bias"]), _ptr(out), Bn, L, D, 1e-6, act, io, _lib.DTYPE_F32, st),
                   "m3_block_act_norm")
        return out, None

    def forward(self, ids: torch.Tensor, mixers=None) -> torch.Tensor:
        """Features (B, L, d_model) float32 of token ids (B, L); ``mixers`` (one per
        block) replace the mixers' forward."""
        x = self.embed[ids].contiguous()
        xin = None
        if self.prenorm and self.blocks:
            b0 = self.blocks[0]
            xin = torch.empty(*x.shape, device=x.device, dtype=self.dtype)
            _lib.check(_lib.load().m3_block_norm(_ptr(x), _ptr(b0["ln_scale"]), _ptr(b0["ln_bias"]), _ptr(xin),
                                                 x.shape[0], x.shape[1], x.shape[2], 1e-6, _IO[self.dtype],
                                                 _stream(x)), "m3_block_norm")
        for i, b in enumerate(self.blocks):
            nxt = self.blocks[i + 1] if i + 1 < len(self.blocks) else None
            x, xin = self._block(b, x, xin, nxt, mixers[i] if mixers else None)
        return x

    def _head(self, x: torch.Tensor) -> torch.Tensor:
        """log_softmax of the decoder Dense on float32 features (..., d_model)."""
        if self.decoder_w is None:
            raise ValueError("the head needs decoder_w and decoder_b in the parameters")
        z = self._decoder(x)
        rows = z.numel() // z.shape[-1]
        _lib.check(_lib.load().m3_log_softmax(_ptr(z), _ptr(z), 1, rows, z.shape[-1], _stream(z)), "m3_log_softmax")
        return z

    def _decoder(self, x: torch.Tensor) -> torch.Tensor:
        """The decoder Dense on float32 features (..., d_model): float32 logits, split-bf16
        products in a bf16 stack."""
        if self._dec_w3 is None:
            return F.linear(x, self.decoder_w, self.decoder_b).contiguous()
        x2 = x.reshape(-1, self.d_model).contiguous()
        z = torch.addmm(self.decoder_b, split_bf16x3(x2), self._dec_w3.t(), out_dtype=torch.float32)
        return z.reshape(*x.shape[:-1], z.shape[-1])

    def prefill(self, ids: torch.Tensor, state=None):
        """Per-token log-probabilities (B, L, vocab) of ids (B, L), continuing each
        block's recurrent carry from ``state`` (a list, one carry per block; None:
        from zero), and the state after the last token, for step() or another prefill
        (the LOB models' generation: prefill, then one token at a time)."""
        new_state = []

        def prefill_mixer(i):
            def run(t):
                out, carry = self.blocks[i]["mixer"].prefill(t, state[i] if state else None)
                new_state.append(carry)
                return out
            return run
        x = self.forward(ids, mixers=[prefill_mixer(i) for i in range(len(self.blocks))])
        return self._head(x), new_state

    def step(self, ids_t: torch.Tensor, state):
        """One token per sequence: ids_t (B,) -> (log-probabilities (B, vocab), state),
        every block's mixer through its decode step (Mamba3Layer.step), the carries
        in ``state`` updated in place."""
        Bn = ids_t.shape[0]

        def step_mixer(i):
            def run(t):
                out, _ = self.blocks[i]["mixer"].step(t.reshape(Bn, self.d_model), state[i])
                return out.reshape(Bn, 1, self.d_model)
            return run
        x = self.forward(ids_t.reshape(Bn, 1), mixers=[step_mixer(i) for i in range(len(self.blocks))])
        return self._head(x)[:, 0], state

    __call__ = forward

    def loss_and_grads(self, ids: torch.Tensor, targets: torch.Tensor):
        """Mean negative log-likelihood of ``targets`` (B, L) under the per-token head
        (log_softmax of the decoder Dense on the features of ``ids``), and its
        gradients, float32, in the layouts of the parameters the stack was built from
        (flax Dense kernels (in, out)): a dict with embed, layers (per block: mixer
        (Mamba3Layer's parameter names), ln_scale, ln_bias, out1_w, out1_b, out2_w,
        out2_b), decoder_w, decoder_b.  Parameters unused by the activation get zero
        gradients.  The weights are the compute-dtype copies taken when the stack was
        built.  Returns (loss (0-d float32 tensor), grads)."""
        if not self.prenorm:
            raise NotImplementedError("loss_and_grads covers prenorm stacks")
        if self.decoder_w is None:
            raise ValueError("loss_and_grads needs decoder_w and decoder_b in the parameters")
        lib, io, dt = _lib.load(), _IO[self.dtype], self.dtype
        Bn, L = ids.shape
        D, V = self.d_model, self.decoder_w.shape[0]
        act = _ACT[self.activation]
        x = self.embed[ids].contiguous()
        st = _stream(x)
        f32 = dict(device=x.device, dtype=torch.float32)
        # ---- forward, keeping each block's intermediates
        b0 = self.blocks[0]
        xin = torch.empty(Bn, L, D, device=x.device, dtype=dt)
        _lib.check(lib.m3_block_norm(_ptr(x), _ptr(b0["ln_scale"]), _ptr(b0["ln_bias"]), _ptr(xin), Bn, L, D, 1e-6, io,
                                     st), "m3_block_norm")
        saves = []
        for i, b in enumerate(self.blocks):
            mixer = b["mixer"]
            y, msaved, _ = mixer._run(xin, mixer.w_in, mixer.w_out, keep=True)
            y = y.contiguous()
            g = h1 = h2 = None
            if self.activation != "gelu":
                g = torch.empty_like(y)
                _lib.check(lib.m3_block_gelu(_ptr(y), _ptr(g), Bn, L, D, io, st), "m3_block_gelu")
                h2 = F.linear(g, b["out2_w"], b["out2_b"])
                if self.activation == "full_glu":
                    h1 = F.linear(g, b["out1_w"], b["out1_b"])
            nxt = self.blocks[i + 1] if i + 1 < len(self.blocks) else None
            out = torch.empty_like(x)
            xn = None
            if nxt is None:
                _lib.check(lib.m3_block_act(_ptr(y), _ptr(h1), _ptr(h2), _ptr(x), _ptr(out), Bn, L, D, act, io, st),
                           "m3_block_act")
            else:
                xn = torch.empty(Bn, L, D, device=x.device, dtype=dt)
                _lib.check(lib.m3_block_act_norm(_ptr(y), _ptr(h1), _ptr(h2), _ptr(x), _ptr(out),
                                                 _ptr(nxt["ln_scale"]), _ptr(nxt["ln_bias"]), _ptr(xn), Bn, L, D,
                                                 1e-6, act, io, io, st), "m3_block_act_norm")
            saves.append(dict(x=x, y=y, g=g, h1=h1, h2=h2, m=msaved))
            x, xin = out, xn
        # ---- the head: loss and, in place, the logits' gradient
        z = self._decoder(x)
        tg = targets.to(device=z.device, dtype=torch.int32).contiguous()
        if tuple(tg.shape) != (Bn, L):
            raise ValueError(f"targets must be {(Bn, L)}, got {tuple(tg.shape)}")
        rows = Bn * L
        loss_rows = torch.empty(rows, **f32)
        _lib.check(lib.m3_log_softmax_nll(_ptr(z), _ptr(tg), _ptr(loss_rows), Bn, L, V, 1.0 / rows, st),
                   "m3_log_softmax_nll")
        loss = loss_rows.sum() / rows
        dz = z.reshape(rows, V)
        x2 = x.reshape(rows, D)
        if self._dec_w3 is None:
            gw = x2.t() @ dz
            dres = (dz @ self.decoder_w).reshape(Bn, L, D)       # the features' gradient, float32
        else:   # split-bf16 products: x_hi dz_hi + x_lo dz_hi + x_hi dz_lo, and dz W likewise
            gw = torch.mm(split_bf16x3(x2, stacked=True, lo_mid=True).t(), split_bf16x3(dz, stacked=True),
                          out_dtype=torch.float32)
            dres = torch.mm(split_bf16x3(dz), self._dec_w3b, out_dtype=torch.float32).reshape(Bn, L, D)
        grads = dict(decoder_w=gw, decoder_b=dz.sum(0))
        # ---- the blocks in reverse
        layers = [None] * len(self.blocks)
        for i in reversed(range(len(self.blocks))):
            sv, b = saves[i], self.blocks[i]
            y = sv["y"]
            lg = dict(out1_w=torch.zeros(D, D, **f32), out1_b=torch.zeros(D, **f32),
                      out2_w=torch.zeros(D, D, **f32), out2_b=torch.zeros(D, **f32))
            dd = torch.empty_like(y)
            dh2 = torch.empty_like(y) if self.activation != "gelu" else None
            _lib.check(lib.m3_block_act_bwd(_ptr(dres), _ptr(y), _ptr(sv["h1"]), _ptr(sv["h2"]), _ptr(dh2), _ptr(dd),
                                            Bn, L, D, act, io, st), "m3_block_act_bwd")
            if self.activation == "gelu":
                dy = dd
            else:
                g2 = sv["g"].reshape(rows, D)
                dg = dh2 @ b["out2_w"]                            # F.linear's (out, in) kernel: dh2 W
                lg["out2_w"] = (g2.t() @ dh2.reshape(rows, D)).float()
                lg["out2_b"] = dh2.reshape(rows, D).sum(0, dtype=torch.float32)
                if self.activation == "full_glu":
                    dg = dg + dd @ b["out1_w"]
                    lg["out1_w"] = (g2.t() @ dd.reshape(rows, D)).float()
                    lg["out1_b"] = dd.reshape(rows, D).sum(0, dtype=torch.float32)
                dy = torch.empty_like(y)
                _lib.check(lib.m3_block_gelu_bwd(_ptr(dg.contiguous()), _ptr(dd), _ptr(y), _ptr(dy), Bn, L, D, act,
                                                 io, st), "m3_block_gelu_bwd")
            mixer = b["mixer"]
            dxin, mgrads = mixer._backward(sv["m"], dy, mixer.w_in, mixer.w_out)
            lg["mixer"] = dict(zip(PARAM_NAMES, mgrads))
            # the prenorm LayerNorm, and the residual path
            dx = torch.empty_like(sv["x"])
            lg["ln_scale"], lg["ln_bias"] = torch.empty(D, **f32), torch.empty(D, **f32)
            ws = torch.empty(max(lib.m3_block_norm_bwd_ws_bytes(Bn, L, D), 16), dtype=torch.uint8, device=x.device)
            _lib.check(lib.m3_block_norm_bwd(_ptr(sv["x"]), _ptr(b["ln_scale"]), _ptr(dxin.contiguous()), _ptr(dres),
                                             _ptr(dx), _ptr(lg["ln_scale"]), _ptr(lg["ln_bias"]), Bn, L, D, 1e-6,
                                             io, ws.data_ptr(), ws.numel(), st), "m3_block_norm_bwd")
            layers[i] = lg
            dres = dx
        grads["layers"] = layers
        grads["embed"] = torch.zeros_like(self.embed).index_add_(0, ids.reshape(-1), dres.reshape(rows, D))
        return loss, grads

    def logits(self, ids: torch.Tensor) -> torch.Tensor:
        """Per-token log-probabilities (B, L, vocab), float32."""
        return self._head(self.forward(ids))

    def step_graph(self, state) -> "StepGraph":
        """``step`` on the carries of ``state`` captured once in a HIP graph (see
        StepGraph): the generation loop's steps then replay it."""
        return StepGraph(self, state)


class StepGraph:
    """Mamba3Stack.step for one batch of carries, captured once in a HIP graph
    (torch.cuda.CUDAGraph): a call copies the token ids (B,) into the graph's input and
    replays every launch of the step (about 300 at config 5: the GEMMs, the layer,
    decode and block kernels, the head) with no host work between them.  It returns
    the log-probabilities (B, vocab) in the graph's output buffer, which the next call
    overwrites, and advances the carries of ``state`` in place, as step does.  The
    decode mode knobs (MAMBA3_RECURRENT_*) are read once, at capture.  Nothing in the
    step records a memset node: the library has none, and its buffers are written
    whole by their kernels."""

    def __init__(self, stack: Mamba3Stack, state):
        dev = state[0][1].device
        B = state[0][1].shape[0]
        self.state = state
        self.ids = torch.zeros(B, dtype=torch.long, device=dev)
        # One eager step first, on copies of the carries, for the libraries' first-call
        # set-up (which capture would not allow); then the capture, which runs nothing.
        cur = torch.cuda.current_stream(dev)
        side = torch.cuda.Stream(dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            stack.step(self.ids, [tuple(t.clone() for t in c) for c in state])
        cur.wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out, _ = stack.step(self.ids, state)

    def __call__(self, ids_t: torch.Tensor) -> torch.Tensor:
        self.ids.copy_(ids_t)
        self.graph.replay()
        return self.out


def split_bf16x3(x: torch.Tensor, stacked: bool = False, lo_mid: bool = False) -> torch.Tensor:
    """The bf16 operand of a split-bf16 product from x (M, K) float32 contiguous, hi =
    bf16(x) and lo = bf16(x - hi) by m3_split_bf16x3: side by side (M, 3K) = [hi | hi |
    lo], or stacked (3M, K) = [hi; hi; lo] ([hi; lo; hi] with lo_mid)."""
    if x.dim() != 2 or x.dtype != torch.float32 or not x.is_contiguous() or not x.is_cuda:
        raise ValueError("split_bf16x3 takes a contiguous 2-D float32 device tensor")
    M, K = x.shape
    if stacked:
        out = torch.empty(3 * M, K, device=x.device, dtype=torch.bfloat16)
        parts, ld = (out[:M], out[M:2 * M], out[2 * M:]), K
    else:
        out = torch.empty(M, 3 * K, device=x.device, dtype=torch.bfloat16)
        parts, ld = (out[:, :K], out[:, K:2 * K], out[:, 2 * K:]), 3 * K
    hi_a, hi_b, lo = (parts[0], parts[2], parts[1]) if lo_mid else parts
    _lib.check(_lib.load().m3_split_bf16x3(_ptr(x), hi_a.data_ptr(), hi_b.data_ptr(), lo.data_ptr(), M, K, ld,
                                           _stream(x)), "m3_split_bf16x3")
    return out


def init_params(vocab: int, d_model: int, n_layers: int, seed: int, device, d_state: int = 128,
                headdim: int = 64) -> Dict:
    """Random float32 parameters on the device (the mixer's with its reference
    initialisers, LayerNorm ones/zeros, Dense kernels N(0, 1/fan_in), the decoder
    Dense to ``vocab``)."""
    from .layer import init_params as mixer_params
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    f = dict(device=device, dtype=torch.float32)
    p = dict(embed=torch.randn(vocab, d_model, generator=g, **f), layers=[])
    for i in range(n_layers):
        lp = dict(mixer=mixer_params(d_model, seed * 1000 + i, device, d_state=d_state, headdim=headdim),
                  ln_scale=torch.ones(d_model, **f), ln_bias=torch.zeros(d_model, **f))
        for n in ("out1", "out2"):
            lp[n + "_w"] = torch.randn(d_model, d_model, generator=g, **f) / d_model ** 0.5
            lp[n + "_b"] = torch.zeros(d_model, **f)
        p["layers"].append(lp)
    p["decoder_w"] = torch.randn(d_model, vocab, generator=g, **f) / d_model ** 0.5
    p["decoder_b"] = torch.zeros(vocab, **f)
    return p
