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
m3_log_softmax (lob_seq_model.py:530-542).
Inference only (dropout is the identity).
"""
from __future__ import annotations

from typing import Dict, List

import torch
import torch.nn.functional as F

from . import _lib
from .layer import Mamba3Layer
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
        if "decoder_w" in params:
            self.decoder_w = params["decoder_w"].float().t().contiguous()
            self.decoder_b = params["decoder_b"].float().contiguous()

    def _block(self, b, x, xin, nxt):
        """SequenceLayer.__call__ (layers.py:108-160) on the float32 residual x (B, L, D).
        Prenorm: xin is this block's normalised input, made by the previous block's
        epilogue (or by m3_block_norm for the first block), and the epilogue makes the
        next block's (nxt) the same way.  Returns (residual, next block's input)."""
        lib, io, st = _lib.load(), _IO[self.dtype], _stream(x)
        Bn, L, D = x.shape
        y = b["mixer"](xin if self.prenorm else x).contiguous()     # compute dtype
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

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
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
            x, xin = self._block(b, x, xin, nxt)
        return x

    __call__ = forward

    def logits(self, ids: torch.Tensor) -> torch.Tensor:
        """Per-token log-probabilities (B, L, vocab), float32."""
        if self.decoder_w is None:
            raise ValueError("logits needs decoder_w and decoder_b in the parameters")
        z = F.linear(self.forward(ids), self.decoder_w, self.decoder_b).contiguous()
        _lib.check(_lib.load().m3_log_softmax(_ptr(z), _ptr(z), z.shape[0], z.shape[1], z.shape[2], _stream(z)),
                   "m3_log_softmax")
        return z


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
