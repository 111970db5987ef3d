"""torch-CPU restatement of the two headline configurations — the CPU BASELINE of bench.py.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): it is the reference CPU path that bench.py's
`cpu_baseline` leg times on the GPU box's host cores, never the measured or shipped path. The
reference's own CPU layers (Accelerate / BNNS behind Swift) cannot be built here, so these are the
same layer definitions written with torch's CPU operators, in fp32:

  * UNetEncoderBlock (UNet.swift:80-100) with the HTDemucs rewrite: reflect padding (k-1)/2
    (DynamicConv1D.swift:288-324) + nn.functional.conv1d, group_norm (1 group, eps 1e-5,
    Normalization.swift:665-724), tanh GELU (Activations.swift:124-137), the 1x1 conv and
    nn.functional.glu over channels (NN.metal:1012-1023);
  * MultiHeadAttention with packed in_proj rows Q;K;V (Attention.swift:840-976), softmax over keys;
  * FeedForward Linear -> tanh GELU -> Linear (Transformer.swift:315-363), layer_norm
    (Normalization.swift:804-879), LayerScale as an elementwise multiply, and the cross-domain
    layer structure of oracle.layers.cross_transformer.

tests/test_oracle.py checks every function here against the numpy oracle.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

__all__ = ["time_encoder", "cross_transformer", "to_torch"]


def to_torch(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def encoder_block(x: torch.Tensor, lv: dict) -> torch.Tensor:
    w = lv["conv.weight"]
    pad = (w.shape[-1] - 1) // 2
    y = F.conv1d(F.pad(x, (pad, pad), mode="reflect"), w, lv["conv.bias"], stride=4)
    y = F.gelu(F.group_norm(y, 1, lv["norm.weight"], lv["norm.bias"], eps=1e-5),
               approximate="tanh")
    return F.glu(F.conv1d(y, lv["rewrite.weight"], lv["rewrite.bias"]), dim=1)


def time_encoder(x: torch.Tensor, levels: list) -> torch.Tensor:
    """Config 4: the chained encoder levels (torch tensors in `levels`)."""
    for lv in levels:
        x = encoder_block(x, lv)
    return x


def mha(xq: torch.Tensor, xkv: torch.Tensor, p: dict, pre: str, heads: int) -> torch.Tensor:
    E = xq.shape[-1]
    hd = E // heads
    w, b = p[pre + "in_proj_weight"], p[pre + "in_proj_bias"]
    q = F.linear(xq, w[:E], b[:E])
    kv = F.linear(xkv, w[E:], b[E:])
    k, v = kv[..., :E], kv[..., E:]
    B, Sq, Sk = xq.shape[0], xq.shape[1], xkv.shape[1]
    q = q.reshape(B, Sq, heads, hd).transpose(1, 2)
    k = k.reshape(B, Sk, heads, hd).transpose(1, 2)
    v = v.reshape(B, Sk, heads, hd).transpose(1, 2)
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * (1.0 / math.sqrt(hd))
    o = torch.matmul(torch.softmax(s, dim=-1), v)
    o = o.transpose(1, 2).reshape(B, Sq, E)
    return F.linear(o, p[pre + "out_proj_weight"], p[pre + "out_proj_bias"])


def _ln(x, p, pre):
    return F.layer_norm(x, (x.shape[-1],), p[pre + ".weight"], p[pre + ".bias"], eps=1e-5)


def _ffn(x, p, pre):
    h = F.gelu(F.linear(x, p[pre + "linear1.weight"], p[pre + "linear1.bias"]),
               approximate="tanh")
    return F.linear(h, p[pre + "linear2.weight"], p[pre + "linear2.bias"])


def cross_transformer(T: torch.Tensor, Fq: torch.Tensor, p: dict, layers: int, heads: int):
    """Config 5: even layers self-attention per branch, odd layers cross-attention on the
    pre-layer states (the structure of oracle.layers.cross_transformer)."""
    for i in range(layers):
        pt, pf = f"layers.{i}.time.", f"layers.{i}.freq."
        if i % 2 == 0:
            out = []
            for X, pre in ((T, pt), (Fq, pf)):
                h = _ln(X, p, pre + "norm1")
                X = X + p[pre + "gamma_1.scale"] * mha(h, h, p, pre + "attn.", heads)
                X = X + p[pre + "gamma_2.scale"] * _ffn(_ln(X, p, pre + "norm2"), p, pre)
                out.append(X)
            T, Fq = out
        else:
            Tn = T + p[pt + "gamma_1.scale"] * mha(_ln(T, p, pt + "norm1"),
                                                   _ln(Fq, p, pt + "norm2"), p, pt + "attn.",
                                                   heads)
            Fn = Fq + p[pf + "gamma_1.scale"] * mha(_ln(Fq, p, pf + "norm1"),
                                                    _ln(T, p, pf + "norm2"), p, pf + "attn.",
                                                    heads)
            Tn = Tn + p[pt + "gamma_2.scale"] * _ffn(_ln(Tn, p, pt + "norm3"), p, pt)
            Fn = Fn + p[pf + "gamma_2.scale"] * _ffn(_ln(Fn, p, pf + "norm3"), p, pf)
            T, Fq = Tn, Fn
    return T, Fq
