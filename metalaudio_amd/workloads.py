"""Seeded synthetic inputs and weights for the five benchmark configurations.

One numpy PCG64 generator per configuration (seeds 1001..1005); every tensor is fp32, drawn
in a fixed order, so the GPU run and the CPU baseline see identical bits. Init rules:
Kaiming-normal conv weights (std = sqrt(2 / fan_in), fan_in = Cin * K), N(0, 0.02) linear and
attention weights, zero biases, norm gamma = 1 and beta = 0, LayerScale 1e-4.

`stress=True` additionally draws non-trivial biases and norm affine parameters (used by the
parity tests so that every parameter path is exercised; the benchmark uses the plain spec).
"""
from __future__ import annotations

import numpy as np

SEEDS = {1: 1001, 2: 1002, 3: 1003, 4: 1004, 5: 1005}

# config 4: HTDemucs time-branch encoder
ENC_CHANNELS = [2, 48, 96, 192, 384]
ENC_KERNEL, ENC_STRIDE = 8, 4
CHUNK_SAMPLES = 343980  # 7.8 s at 44.1 kHz

# config 5: cross-domain transformer
T5_EMBED, T5_HEADS, T5_FFN, T5_LAYERS, T5_LAYERSCALE = 384, 8, 1536, 5, 1e-4
T5_TIME_LEN, T5_FREQ_LEN, T5_BATCH = 1344, 2688, 4


def _rng(cfg: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(SEEDS[cfg]))


def _kaiming(rng, shape, fan_in):
    return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def _normal(rng, shape, std):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def _affine(rng, n, stress):
    if not stress:
        return np.ones(n, np.float32), np.zeros(n, np.float32)
    return (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32), \
        (0.1 * rng.standard_normal(n)).astype(np.float32)


def _bias(rng, n, stress, scale=0.05):
    if not stress:
        return np.zeros(n, np.float32)
    return (scale * rng.standard_normal(n)).astype(np.float32)


def config1(stress: bool = False) -> dict:
    """Conv1D 2->48 k8 s4 pad 0 -> GroupNorm(1) -> GELU on [1, 2, 44100]."""
    r = _rng(1)
    x = r.uniform(-1.0, 1.0, (1, 2, 44100)).astype(np.float32)
    w = _kaiming(r, (48, 2, 8), 2 * 8)
    b = _bias(r, 48, stress)
    g, be = _affine(r, 48, stress)
    return {"x": x, "conv_w": w, "conv_b": b, "gn_w": g, "gn_b": be, "stride": 4, "padding": 0}


def config2(stress: bool = False) -> dict:
    """Linear 512 -> 2048 on X [2048, 512], then LayerNorm over 2048."""
    r = _rng(2)
    x = r.standard_normal((2048, 512)).astype(np.float32)
    w = _normal(r, (2048, 512), 0.02)
    b = _bias(r, 2048, stress)
    g, be = _affine(r, 2048, stress)
    return {"x": x, "w": w, "b": b, "ln_w": g, "ln_b": be}


def _attn_params(r, E, stress):
    return {
        "in_proj_weight": _normal(r, (3 * E, E), 0.02),
        "in_proj_bias": _bias(r, 3 * E, stress, 0.02),
        "out_proj_weight": _normal(r, (E, E), 0.02),
        "out_proj_bias": _bias(r, E, stress, 0.02),
    }


def _ffn_params(r, E, Hd, stress):
    return {
        "linear1.weight": _normal(r, (Hd, E), 0.02),
        "linear1.bias": _bias(r, Hd, stress, 0.02),
        "linear2.weight": _normal(r, (E, Hd), 0.02),
        "linear2.bias": _bias(r, E, stress, 0.02),
    }


def config3(stress: bool = False, seq: int = 2048) -> dict:
    """Pre-norm MHSA (E 512, H 8) + FFN 512->2048->512 on x [seq, 512]."""
    r = _rng(3)
    E, Hd = 512, 2048
    x = r.standard_normal((seq, E)).astype(np.float32)
    p = {}
    p["norm1.weight"], p["norm1.bias"] = _affine(r, E, stress)
    for k, v in _attn_params(r, E, stress).items():
        p["attn." + k] = v
    p["norm2.weight"], p["norm2.bias"] = _affine(r, E, stress)
    p.update(_ffn_params(r, E, Hd, stress))
    return {"x": x, "params": p, "embed": E, "heads": 8, "ffn": Hd}


def config4(stress: bool = False, samples: int = CHUNK_SAMPLES, batch: int = 1) -> dict:
    """4-level time encoder: k8 s4 reflect-3 conv, GN(1), GELU, 1x1 C->2C, GLU."""
    r = _rng(4)
    x = r.uniform(-1.0, 1.0, (batch, 2, samples)).astype(np.float32)
    levels = []
    for cin, cout in zip(ENC_CHANNELS[:-1], ENC_CHANNELS[1:]):
        lv = {
            "conv.weight": _kaiming(r, (cout, cin, ENC_KERNEL), cin * ENC_KERNEL),
            "conv.bias": _bias(r, cout, stress),
        }
        lv["norm.weight"], lv["norm.bias"] = _affine(r, cout, stress)
        lv["rewrite.weight"] = _kaiming(r, (2 * cout, cout, 1), cout)
        lv["rewrite.bias"] = _bias(r, 2 * cout, stress)
        levels.append(lv)
    return {"x": x, "levels": levels}


def cross_encoder_metalnn(batch: int, time_len: int, freq_len: int, embed: int, heads: int,
                          ffn: int, layers: int, seed: int = 1006) -> dict:
    """Inputs and weights for the reference-structured CrossTransformerEncoder (every layer self +
    cross + FFN per branch), reference names (TransformerLayer.loadWeights), projections scaled
    by 1/sqrt(fan_in) so that every sub-block's update is of the order of its input."""
    r = np.random.Generator(np.random.PCG64(seed))
    E = embed

    def w(shape, fan_in):
        return (r.standard_normal(shape) / np.sqrt(fan_in)).astype(np.float32)

    def b(n):
        return (0.1 * r.standard_normal(n)).astype(np.float32)
    p = {}
    for i in range(layers):
        L = f"layers.{i}."
        for n in ("norm_time_self", "norm_freq_self", "norm_time_cross", "norm_freq_cross",
                  "norm_time_ffn", "norm_freq_ffn"):
            p[L + n + ".weight"] = (1.0 + 0.1 * r.standard_normal(E)).astype(np.float32)
            p[L + n + ".bias"] = b(E)
        for a in ("self_attn_time", "self_attn_freq", "cross_attn_time", "cross_attn_freq"):
            p[L + a + ".in_proj_weight"] = w((3 * E, E), E)
            p[L + a + ".in_proj_bias"] = b(3 * E)
            p[L + a + ".out_proj.weight"] = w((E, E), E)
            p[L + a + ".out_proj.bias"] = b(E)
        for f in ("ffn_time", "ffn_freq"):
            p[L + f + ".linear1.weight"] = w((ffn, E), E)
            p[L + f + ".linear1.bias"] = b(ffn)
            p[L + f + ".linear2.weight"] = w((E, ffn), ffn)
            p[L + f + ".linear2.bias"] = b(E)
    return {"time": r.standard_normal((batch, time_len, E)).astype(np.float32),
            "freq": r.standard_normal((batch, freq_len, E)).astype(np.float32),
            "params": p, "embed": E, "heads": heads, "ffn": ffn, "layers": layers}


def config5(stress: bool = False, batch: int = T5_BATCH, time_len: int = T5_TIME_LEN,
            freq_len: int = T5_FREQ_LEN, layers: int = T5_LAYERS, embed: int = T5_EMBED,
            heads: int = T5_HEADS, ffn: int = T5_FFN) -> dict:
    """Cross-domain bottleneck: E 384, H 8, FFN 1536, LayerScale 1e-4, self/cross alternating
    (other widths for tests)."""
    r = _rng(5)
    E, Hd = embed, ffn
    t = r.standard_normal((batch, time_len, E)).astype(np.float32)
    f = r.standard_normal((batch, freq_len, E)).astype(np.float32)
    p = {}
    for i in range(layers):
        cross = i % 2 == 1
        for br in ("time", "freq"):
            pre = f"layers.{i}.{br}."
            norms = ("norm1", "norm2", "norm3") if cross else ("norm1", "norm2")
            for n in norms:
                p[pre + n + ".weight"], p[pre + n + ".bias"] = _affine(r, E, stress)
            for k, v in _attn_params(r, E, stress).items():
                p[pre + "attn." + k] = v
            for k, v in _ffn_params(r, E, Hd, stress).items():
                p[pre + k] = v
            ls = T5_LAYERSCALE
            p[pre + "gamma_1.scale"] = np.full(E, ls, np.float32) if not stress else \
                (ls * (1.0 + 0.1 * r.standard_normal(E))).astype(np.float32)
            p[pre + "gamma_2.scale"] = np.full(E, ls, np.float32) if not stress else \
                (ls * (1.0 + 0.1 * r.standard_normal(E))).astype(np.float32)
    return {"time": t, "freq": f, "params": p, "embed": E, "heads": heads, "ffn": Hd,
            "layers": layers, "layer_scale": T5_LAYERSCALE}
