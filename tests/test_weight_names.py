"""Weight-name conventions of the C ABI (WeightNameMapper.swift:7-422), host-only. Known answers
are worked out by hand from the reference's naming table (docs/guides/SAFETENSORS_GUIDE.md:180-190)
and doc examples; a generated corpus then checks the library against the oracle's restatement,
including replace-all and non-overlapping-match behaviour."""
import itertools
import json
import struct

import numpy as np
import pytest

from metalaudio_amd import nn
from oracle import weight_names as ow

KNOWN = [
    ("tencoder.0.conv.weight", "time_encoder.0.conv.weight"),
    ("tencoder.2.norm1.bias", "time_encoder.2.norm.bias"),
    ("tdecoder.1.conv_tr.weight", "time_decoder.1.conv_transpose.weight"),
    ("tdecoder.1.norm2.weight", "time_decoder.1.norm.weight"),
    ("encoder.3.conv.weight", "freq_encoder.3.conv.weight"),
    ("encoder.0.norm1.weight", "freq_encoder.0.norm.weight"),
    ("encoder.0.rewrite.weight", "freq_encoder.0.rewrite.weight"),
    ("decoder.2.conv_tr.bias", "freq_decoder.2.conv_transpose.bias"),
    ("channel_upsampler.weight", "freq_to_transformer.weight"),
    ("channel_downsampler.bias", "transformer_to_freq.bias"),
    ("channel_upsampler_t.weight", "time_to_transformer.weight"),
    ("channel_downsampler_t.bias", "transformer_to_time.bias"),
    ("crosstransformer.layers.0.self_attn.in_proj_weight",
     "cross_transformer.layers.0.self_attn_freq.in_proj_weight"),
    ("crosstransformer.layers_t.2.cross_attn.out_proj.weight",
     "cross_transformer.layers.2.cross_attn_time.out_proj.weight"),
    ("crosstransformer.layers.1.linear2.bias", "cross_transformer.layers.1.ffn_freq.linear2.bias"),
    ("crosstransformer.layers_t.0.norm3.weight", "cross_transformer.layers.0.norm3_time.weight"),
    ("crosstransformer.layers.4.norm1.bias", "cross_transformer.layers.4.norm1_freq.bias"),
    # an unrecognised sub-layer gets the path as a suffix of the whole remainder
    ("crosstransformer.layers.0.gamma_1.scale", "cross_transformer.layers.0.gamma_1.scale_freq"),
    ("crosstransformer.norm_in.weight", "cross_transformer.norm_in.weight"),
    ("crosstransformer.layers_t.3", "cross_transformer.layers_t.3"),  # no sub-layer: unchanged
    ("freq_emb.embedding.weight", "freq_emb.embedding.weight"),
    # every occurrence is replaced ...
    ("encoder.1.subencoder.w", "freq_encoder.1.subfreq_encoder.w"),
    # ... left to right without overlap: the second ".norm2." shares its dot with the first
    ("tdecoder.0.norm2.norm2.w", "time_decoder.0.norm.norm2.w"),
    ("tdecoder.0.norm2..norm2.w", "time_decoder.0.norm..norm.w"),
]

REVERSE = [
    ("time_encoder.0.conv.weight", "tencoder.0.conv.weight"),
    ("time_encoder.0.norm.weight", "tencoder.0.norm1.weight"),
    ("time_decoder.1.conv_transpose.weight", "tdecoder.1.conv_tr.weight"),
    ("time_decoder.1.norm.bias", "tdecoder.1.norm2.bias"),
    ("freq_decoder.0.norm.weight", "decoder.0.norm2.weight"),
    ("time_to_transformer.weight", "channel_upsampler_t.weight"),
    # cross-transformer sub-layers are not reverse-mapped (WeightNameMapper.swift:335-340)
    ("cross_transformer.layers.0.self_attn_freq.in_proj_weight",
     "crosstransformer.layers.0.self_attn_freq.in_proj_weight"),
    ("something.else", "something.else"),
]


@pytest.mark.parametrize("src,want", KNOWN)
def test_demucs_to_metalaudio_known_answers(src, want):
    assert ow.demucs_to_metalaudio(src) == want
    assert nn.WeightNameMapper("demucs").to_metalaudio(src) == want
    # mappers of the other conventions leave names alone
    assert nn.WeightNameMapper("metalaudio").to_metalaudio(src) == src
    assert nn.WeightNameMapper("unknown").to_metalaudio(src) == src


@pytest.mark.parametrize("src,want", REVERSE)
def test_metalaudio_to_demucs_known_answers(src, want):
    assert ow.metalaudio_to_demucs(src) == want
    assert nn.WeightNameMapper.from_metalaudio(src, "demucs") == want
    assert nn.WeightNameMapper.from_metalaudio(src, "metalaudio") == src


@pytest.mark.parametrize("names,want", [
    ([], "unknown"),
    (["tencoder.0.conv.weight"], "unknown"),  # score 2 < 3
    (["tencoder.0.conv.weight", "tencoder.0.norm1.weight"], "demucs"),  # 2 + 3
    (["time_encoder.0.conv.weight"], "unknown"),
    (["time_encoder.0.conv.weight", "cross_transformer.layers.0.self_attn_freq.w"],
     "metalaudio"),  # 2 + 3
    (["tencoder.0.x", "a.norm1.b", "time_encoder.0.x", "a.conv_transpose.b"], "unknown"),  # 3 = 3
    (["channel_upsampler.weight", "channel_downsampler.weight", "x.conv_tr.y"], "demucs"),
    (["time_to_transformer.w", "transformer_to_freq.w", "q.self_attn_time.w"], "metalaudio"),
])
def test_detection_known_answers(names, want):
    code = {"metalaudio": ow.METALAUDIO, "demucs": ow.DEMUCS, "unknown": ow.UNKNOWN}[want]
    assert ow.detect(names) == code
    assert nn.WeightNameMapper.detect_convention(names) == want
    assert nn.WeightNameMapper(tensor_names=names).convention == want


def corpus():
    heads = ["tencoder.", "tdecoder.", "encoder.", "decoder.", "crosstransformer.",
             "channel_upsampler.", "channel_downsampler.", "channel_upsampler_t.",
             "channel_downsampler_t.", "time_encoder.", "time_decoder.", "freq_encoder.",
             "freq_decoder.", "cross_transformer.", "freq_to_transformer.",
             "transformer_to_freq.", "time_to_transformer.", "transformer_to_time.", "x."]
    mids = ["0.", "12.", "layers.3.", "layers_t.1.", "layers_t.x.", "layers_t.", "layers.",
            "norm1.", "norm2.", "conv_tr.", "conv_transpose.", "norm.", "encoder.", ""]
    tails = ["self_attn.in_proj_weight", "cross_attn.out_proj.bias", "linear1.weight",
             "linear2.bias", "norm1.weight", "norm2.bias", "norm3.weight", "gamma_1.scale",
             "conv.weight", "norm1.norm1.w", "weight", "", "conv_tr.norm2.b",
             "crosstransformer.layers_t.0.q"]
    return ["".join(p) for p in itertools.product(heads, mids, mids[:6], tails)]


def test_library_matches_oracle_on_generated_corpus():
    names = corpus()
    assert len(names) > 10000
    dm = nn.WeightNameMapper("demucs")
    for n in names:
        assert dm.to_metalaudio(n) == ow.demucs_to_metalaudio(n), n
        assert nn.WeightNameMapper.from_metalaudio(n, "demucs") == ow.metalaudio_to_demucs(n), n
        assert nn.WeightNameMapper.is_metalaudio_naming(n) == ow.is_metalaudio(n), n
        assert nn.WeightNameMapper.is_demucs_naming(n) == ow.is_demucs(n), n
    rng = np.random.default_rng(5)
    for _ in range(300):
        pick = [names[i] for i in rng.integers(0, len(names), rng.integers(0, 6))]
        want = {0: "metalaudio", 1: "demucs", 2: "unknown"}[ow.detect(pick)]
        assert nn.WeightNameMapper.detect_convention(pick) == want, pick


def test_encoder_decoder_names_round_trip():
    """For encoder / decoder / projection names without doubled patterns the two directions are
    inverse (the cross-transformer is one-way by design)."""
    for lvl in range(4):
        for n in (f"tencoder.{lvl}.conv.weight", f"tencoder.{lvl}.norm1.bias",
                  f"tdecoder.{lvl}.conv_tr.weight", f"tdecoder.{lvl}.norm2.weight",
                  f"encoder.{lvl}.rewrite.bias", f"decoder.{lvl}.conv_tr.bias",
                  "channel_upsampler_t.weight", "channel_downsampler.bias"):
            m = ow.demucs_to_metalaudio(n)
            assert nn.WeightNameMapper.is_metalaudio_naming(m) or m.startswith("transformer_to_")
            assert nn.WeightNameMapper.from_metalaudio(m, "demucs") == n


def write_st(path, names):
    header, blobs, off = {}, [], 0
    for i, n in enumerate(names):
        raw = np.full(2, i, np.float32).tobytes()
        header[n] = {"dtype": "F32", "shape": [2], "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_safetensors_mapped_loading(tmp_path):
    """createWeightMapper + loadTensorMapped (WeightNameMapper.swift:393-420) on a Demucs-named
    file: the reverse-mapped name is tried first, then every name is mapped forward."""
    names = ["tencoder.0.conv.weight", "tencoder.0.norm1.weight", "tdecoder.0.conv_tr.weight",
             "crosstransformer.layers.0.self_attn.in_proj_weight",
             "crosstransformer.layers_t.0.linear1.weight"]
    p = tmp_path / "d.safetensors"
    write_st(p, names)
    st = nn.SafeTensors(p)
    m = st.create_weight_mapper()
    assert m.convention == "demucs"
    srt = sorted(names)
    for want in ["time_encoder.0.norm.weight", "time_decoder.0.conv_transpose.weight",
                 "cross_transformer.layers.0.self_attn_freq.in_proj_weight",
                 "cross_transformer.layers.0.ffn_time.linear1.weight"]:
        orig = ow.find_mapped(names, ow.DEMUCS, want)
        assert orig is not None and st.mapped_name(want, m) == orig
        np.testing.assert_array_equal(st.load_tensor_mapped(want, m),
                                      np.full(2, names.index(orig), np.float32))
    with pytest.raises(nn.MNNError) as e:
        st.mapped_name("time_encoder.9.conv.weight", m)
    assert e.value.code == 15
    # a MetalAudio mapper uses names as they are
    ma = nn.WeightNameMapper("metalaudio")
    assert st.mapped_name("tencoder.0.conv.weight", ma) == "tencoder.0.conv.weight"
    with pytest.raises(nn.MNNError):
        st.mapped_name("time_encoder.0.conv.weight", ma)
    assert srt == st.available_tensors


def test_invalid_convention_and_small_buffer():
    import ctypes as C
    from metalaudio_amd._lib import check, lib
    buf = C.create_string_buffer(8)
    with pytest.raises(nn.MNNError) as e:
        check(lib().mnn_weight_name_to_metalaudio(7, b"tencoder.0.w", buf, len(buf)))
    assert e.value.code == 12
    with pytest.raises(nn.MNNError) as e:
        check(lib().mnn_weight_name_to_metalaudio(1, b"tencoder.0.w", buf, len(buf)))
    assert e.value.code == 2
    with pytest.raises(ValueError):
        nn.WeightNameMapper("caffe")
