"""Numpy restatement of the Mamba3 backbone around the mixer (CPU oracle, test-only).

StackedEncoderModel (src/base_model/models/seq_model.py:47-118) with
use_embed_layer=True: nn.Embed, then n_layers SequenceLayer blocks
(layers.py:108-160) whose mixer is Mamba3SSM (oracle.mamba3_layer).  A block is
    skip = x; x = LayerNorm(x) if prenorm; x = mixer(x); activation; x = skip + x;
    x = LayerNorm(x) if not prenorm
with flax defaults: LayerNorm eps 1e-6 with scale and bias, nn.gelu the tanh
approximation, Dense layers with bias; dropout is the identity at inference.
Activations: gelu, full_glu (out1(g) * sigmoid(out2(g)), g = gelu(x)),
half_glu1 (g * sigmoid(out2(g))), half_glu2 (x * sigmoid(out2(g))).  The
per-token head (lm_forward) is the LOB models' decoder in mode "none":
Dense(d_output) on the features, then log_softmax in float32
(lob_seq_model.py:530-542).  Pinned by tests/test_oracle_layer.py.
"""
from __future__ import annotations

import math

import numpy as np

from . import inputs as I
from . import mamba3_layer as ML

LN_EPS = 1e-6
ACTIVATIONS = ("gelu", "full_glu", "half_glu1", "half_glu2")


def layernorm(x, scale, bias, eps=LN_EPS):
    """flax nn.LayerNorm over the last axis."""
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * scale + bias


def gelu(x):
    """flax nn.gelu (approximate=True): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def init_params(vocab, d_model, n_layers, seed, d_state=128, headdim=64):
    """Embedding N(0, 1) (flax Embed's variance-scaled normal, up to scale), per block
    the mixer's parameters (oracle.mamba3_layer.init_params), LayerNorm scale/bias
    and the GLU Dense layers (kernels N(0, 1/fan_in), biases)."""
    rng = np.random.default_rng(seed)
    f = np.float32
    p = dict(embed=rng.standard_normal((vocab, d_model)).astype(f), layers=[])
    for i in range(n_layers):
        lp = dict(mixer=ML.init_params(d_model, seed * 1000 + i, d_state=d_state, headdim=headdim),
                  ln_scale=(1 + 0.1 * rng.standard_normal(d_model)).astype(f),
                  ln_bias=(0.1 * rng.standard_normal(d_model)).astype(f))
        for name in ("out1", "out2"):
            lp[name + "_w"] = (rng.standard_normal((d_model, d_model)) / math.sqrt(d_model)).astype(f)
            lp[name + "_b"] = (0.1 * rng.standard_normal(d_model)).astype(f)
        p["layers"].append(lp)
    p["decoder_w"] = (rng.standard_normal((d_model, vocab)) / math.sqrt(d_model)).astype(f)
    p["decoder_b"] = (0.1 * rng.standard_normal(vocab)).astype(f)
    return p


def block_forward(lp, x, activation, prenorm, d_state, headdim, bf16):
    """SequenceLayer.__call__ (layers.py:108-160) with the Mamba3 mixer."""
    r = (lambda a: np.asarray(I.bf16_round(np.asarray(a, np.float32)), np.float64)) if bf16 else (lambda a: a)
    skip = x
    if prenorm:
        x = layernorm(x, lp["ln_scale"], lp["ln_bias"])
    x = ML.layer_forward(lp["mixer"], x, d_state=d_state, headdim=headdim, bf16=bf16)
    dense = lambda a, n: r(r(a) @ r(lp[n + "_w"]) + lp[n + "_b"])      # noqa: E731  (Dense in the layer dtype)
    if activation == "gelu":
        x = r(gelu(x))
    elif activation == "full_glu":
        g = r(gelu(x))
        x = r(dense(g, "out1") * sigmoid(dense(g, "out2")))
    elif activation == "half_glu1":
        g = r(gelu(x))
        x = r(g * sigmoid(dense(g, "out2")))
    elif activation == "half_glu2":
        g = r(gelu(x))
        x = r(x * sigmoid(dense(g, "out2")))
    else:
        raise ValueError(f"activation must be one of {ACTIVATIONS}")
    x = skip + x
    if not prenorm:
        x = layernorm(x, lp["ln_scale"], lp["ln_bias"])
    return x


def stack_forward(p, ids, activation="half_glu1", prenorm=True, d_state=128, headdim=64, bf16=False):
    """StackedEncoderModel.__call__ (seq_model.py:96-118) on token ids (B, L) ->
    features (B, L, d_model), float64."""
    x = p["embed"][ids].astype(np.float64)
    for lp in p["layers"]:
        x = block_forward(lp, x, activation, prenorm, d_state, headdim, bf16)
    return x


def log_softmax(x):
    m = x.max(-1, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(-1, keepdims=True))


def lm_forward(p, ids, activation="half_glu1", prenorm=True, d_state=128, headdim=64, bf16=False):
    """Per-token log-probabilities (B, L, vocab): the decoder Dense (float32
    parameters on the float32 features) and log_softmax (lob_seq_model.py:530-542)."""
    x = stack_forward(p, ids, activation, prenorm, d_state, headdim, bf16)
    return log_softmax(x @ p["decoder_w"].astype(np.float64) + p["decoder_b"])
