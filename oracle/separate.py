"""numpy restatement of time-domain HTDemucs separation and the long-audio segment driver
(reference: zkeown/MetalAudio, Sources/MetalNN/HTDemucs.swift and
docs/guides/HTDEMUCS_GUIDE.md).

TEST INFRASTRUCTURE ONLY — see oracle/__init__.py.
"""
from __future__ import annotations

import numpy as np

from .layers import conv1d, decoder_block, encoder_block, unet_padding

__all__ = ["separate_time", "separate_long"]


def separate_time(x, params, cfg, dtype=np.float64):
    """HTDemucs.separate(input:mode: .timeOnly) (HTDemucs.swift:617-691): de-interleave, UNet
    zero padding (left half rounded down), encoders (GroupNorm min(groups, C) at level 0,
    :260-276) keeping each output as the skip, decoders from the deepest level (:279-292,
    forwardTimeUNet :521-548), one 1x1 conv head per stem (:333-350, :376-392), crop and
    interleave. x [n * C]; returns [stems, n * C]."""
    C, ch, ng = cfg["input_channels"], list(cfg["channels"]), cfg["num_groups"]
    k, s, levels = cfg["kernel_size"], cfg["stride"], len(ch)
    x = np.asarray(x, dtype=dtype)
    n = x.shape[0] // C
    lp, _, Lp = unet_padding(n, levels, k, s)
    xp = np.zeros((C, Lp), dtype=dtype)
    xp[:, lp:lp + n] = x.reshape(n, C).T
    chans = [C] + ch
    y, skips = xp, []
    for i in range(levels):
        p = params[f"time_encoder.{i}"]
        g = min(ng, chans[i]) if i == 0 else ng
        y = encoder_block(y, p["conv.weight"], p["conv.bias"], p["norm.weight"], p["norm.bias"],
                          g, k, s, dtype=dtype)
        skips.append(y)
    for j in range(levels):
        i = levels - 1 - j
        co = C if i == 0 else chans[i]
        g = max(1, min(ng, co) if i == 0 else ng)
        p = params[f"time_decoder.{j}"]
        y = decoder_block(y, skips[i], p["conv_transpose.weight"], p["conv_transpose.bias"],
                          p["norm.weight"], p["norm.bias"], g, k, s, dtype=dtype)
    out = []
    for h in range(cfg["num_stems"]):
        p = params[f"output_heads.{h}"]
        st = conv1d(y, p["weight"], p["bias"], dtype=dtype)
        out.append(st[:, lp:lp + n].T.reshape(-1))
    return np.stack(out)


def separate_long(x, C, segment, overlap, segment_fn, dtype=np.float64):
    """Segments of `segment` frames every segment - overlap frames (HTDEMUCS_GUIDE.md:170-191);
    segment_fn maps interleaved [len * C] to [stems, len * C]. The first F frames a segment shares
    with the previous one blend linearly, new weight (i + 1) / (F + 1); the rest is written as
    is. segment <= 0 or >= n: one call."""
    x = np.asarray(x, dtype=dtype)
    n = x.shape[0] // C
    if segment <= 0 or segment >= n:
        return segment_fn(x)
    out, prev_end, start = None, 0, 0
    while start < n:
        end = min(start + segment, n)
        y = segment_fn(x[start * C:end * C])
        if out is None:
            out = np.zeros((y.shape[0], n * C), dtype=dtype)
        fade = max(0, prev_end - start)
        yf = y.reshape(y.shape[0], end - start, C)
        of = out.reshape(out.shape[0], n, C)
        w = ((np.arange(fade) + 1) / (fade + 1))[None, :, None]
        of[:, start:start + fade] = of[:, start:start + fade] * (1 - w) + yf[:, :fade] * w
        of[:, start + fade:end] = yf[:, fade:]
        prev_end = end
        if end == n:
            break
        start += segment - overlap
    return out
