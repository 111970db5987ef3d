"""Python restatement of the weight-name conventions (reference: zkeown/MetalAudio,
Sources/MetalNN/WeightNameMapper.swift). Plain string rules: `str.replace` replaces every
occurrence, as Foundation's replacingOccurrences does.

TEST INFRASTRUCTURE ONLY — see oracle/__init__.py.
"""
from __future__ import annotations

import re

__all__ = ["METALAUDIO", "DEMUCS", "UNKNOWN", "detect", "demucs_to_metalaudio",
           "metalaudio_to_demucs", "is_metalaudio", "is_demucs", "find_mapped"]

METALAUDIO, DEMUCS, UNKNOWN = 0, 1, 2


def detect(names) -> int:
    """detectConvention(from:) (WeightNameMapper.swift:83-137)."""
    d = m = 0
    for n in names:
        d += 2 * (n.startswith("tencoder.") or n.startswith("tdecoder."))
        d += 2 * n.startswith("crosstransformer.")
        d += ".conv_tr." in n
        d += (".norm1." in n) or (".norm2." in n)
        d += n.startswith("channel_upsampler.") or n.startswith("channel_downsampler.")
        m += 2 * (n.startswith("time_encoder.") or n.startswith("time_decoder."))
        m += 2 * (n.startswith("freq_encoder.") or n.startswith("freq_decoder."))
        m += 2 * n.startswith("cross_transformer.")
        m += ".conv_transpose." in n
        m += ("_to_transformer." in n) or ("transformer_to_" in n)
        m += (".self_attn_freq." in n) or (".self_attn_time." in n)
    if m > d and m >= 3:
        return METALAUDIO
    if d > m and d >= 3:
        return DEMUCS
    return UNKNOWN


def _sublayer(sub: str, path: str) -> str:
    """remapTransformerSublayer (:258-295)."""
    for stem in ("self_attn", "cross_attn"):
        if sub.startswith(stem + "."):
            return f"{stem}_{path}." + sub[len(stem) + 1:]
    if sub.startswith("linear1.") or sub.startswith("linear2."):
        return f"ffn_{path}.{sub}"
    for stem in ("norm1", "norm2", "norm3"):
        if sub.startswith(stem + "."):
            return f"{stem}_{path}." + sub[len(stem) + 1:]
    return f"{sub}_{path}"


def _cross(name: str) -> str:
    """remapCrossTransformerName (:225-255): once the layers_t pattern occurs anywhere, the level
    is read right after the fixed prefix at the start of the name."""
    if re.search(r"cross_transformer\.layers_t\.([0-9]+)\.", name):
        prefix, path = "cross_transformer.layers_t.", "time"
    elif name.startswith("cross_transformer.layers.") and ".layers_t." not in name:
        prefix, path = "cross_transformer.layers.", "freq"
    else:
        return name
    after = name[len(prefix):]
    if "." not in after:
        return name
    level, rest = after.split(".", 1)
    return f"cross_transformer.layers.{level}.{_sublayer(rest, path)}"


def demucs_to_metalaudio(n: str) -> str:
    """demucsToMetalAudio (:177-222)."""
    if n.startswith("tencoder."):
        return n.replace("tencoder.", "time_encoder.").replace(".norm1.", ".norm.")
    if n.startswith("tdecoder."):
        n = n.replace("tdecoder.", "time_decoder.")
        return n.replace(".conv_tr.", ".conv_transpose.").replace(".norm2.", ".norm.")
    if n.startswith("encoder."):
        return n.replace("encoder.", "freq_encoder.").replace(".norm1.", ".norm.")
    if n.startswith("decoder."):
        n = n.replace("decoder.", "freq_decoder.")
        return n.replace(".conv_tr.", ".conv_transpose.").replace(".norm2.", ".norm.")
    for old, new in (("channel_upsampler.", "freq_to_transformer."),
                     ("channel_downsampler.", "transformer_to_freq."),
                     ("channel_upsampler_t.", "time_to_transformer."),
                     ("channel_downsampler_t.", "transformer_to_time.")):
        if n.startswith(old):
            return n.replace(old, new)
    if n.startswith("crosstransformer."):
        return _cross(n.replace("crosstransformer.", "cross_transformer."))
    return n


def metalaudio_to_demucs(n: str) -> str:
    """metalAudioToDemucs (:300-342); cross-transformer sub-layers are not reverse-mapped."""
    if n.startswith("time_encoder."):
        return n.replace("time_encoder.", "tencoder.").replace(".norm.", ".norm1.")
    if n.startswith("time_decoder."):
        n = n.replace("time_decoder.", "tdecoder.")
        return n.replace(".conv_transpose.", ".conv_tr.").replace(".norm.", ".norm2.")
    if n.startswith("freq_encoder."):
        return n.replace("freq_encoder.", "encoder.").replace(".norm.", ".norm1.")
    if n.startswith("freq_decoder."):
        n = n.replace("freq_decoder.", "decoder.")
        return n.replace(".conv_transpose.", ".conv_tr.").replace(".norm.", ".norm2.")
    for old, new in (("freq_to_transformer.", "channel_upsampler."),
                     ("transformer_to_freq.", "channel_downsampler."),
                     ("time_to_transformer.", "channel_upsampler_t."),
                     ("transformer_to_time.", "channel_downsampler_t."),
                     ("cross_transformer.", "crosstransformer.")):
        if n.startswith(old):
            return n.replace(old, new)
    return n


def is_metalaudio(n: str) -> bool:
    """isMetalAudioNaming (:372-380)."""
    return n.startswith(("time_encoder.", "time_decoder.", "freq_encoder.", "freq_decoder.",
                         "cross_transformer.", "time_to_transformer.", "freq_to_transformer."))


def is_demucs(n: str) -> bool:
    """isDemucsNaming (:383-388)."""
    return n.startswith(("tencoder.", "tdecoder.", "crosstransformer.", "channel_upsampler."))


def find_mapped(available, conv: int, name: str):
    """loadTensorMapped's lookup (:404-420); None when the tensor is absent."""
    avail = sorted(available)
    if conv == METALAUDIO:
        return name if name in avail else None
    orig = metalaudio_to_demucs(name) if conv == DEMUCS else name
    if orig in avail:
        return orig
    for n in avail:
        if (demucs_to_metalaudio(n) if conv == DEMUCS else n) == name:
            return n
    return None
