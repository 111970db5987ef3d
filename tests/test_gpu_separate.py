"""GPU parity of time-domain separation and the long-audio driver through the C ABI against the
oracle (oracle/separate.py): one pass (HTDemucs.separate .timeOnly) and segmented runs with
crossfades (overlaps, zero overlap, a short last segment, a segment covering everything).

fp32 bar: |gpu - oracle| <= 1e-4 + 1e-3 * |oracle| per element."""
import sys

import numpy as np
import pytest

from metalaudio_amd import nn
from oracle import separate as osep
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(81)


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    return nn.AudioDevice(0)


@pytest.fixture(scope="module")
def stream(dev):
    return nn.Stream(dev)


def model(levels=3, seed=5):
    r = np.random.default_rng(seed)
    ch = [16, 32, 64][:levels]
    cfg = {"input_channels": 2, "num_stems": 4, "channels": ch, "kernel_size": 8, "stride": 4,
           "num_groups": 4}
    chans = [2] + ch
    P = {}
    for i in range(levels):
        ci, co = chans[i], chans[i + 1]
        P[f"time_encoder.{i}"] = {
            "conv.weight": (r.standard_normal((co, ci, 8)) * np.sqrt(2 / (8 * ci))),
            "conv.bias": r.standard_normal(co) * 0.1, "norm.weight": 1 + 0.1 * r.standard_normal(co),
            "norm.bias": 0.1 * r.standard_normal(co)}
    for j in range(levels):
        i = levels - 1 - j
        ci, co = chans[i + 1], (2 if i == 0 else chans[i])
        P[f"time_decoder.{j}"] = {
            "conv_transpose.weight": r.standard_normal((2 * ci, co, 8)) * np.sqrt(1 / (4 * ci)),
            "conv_transpose.bias": r.standard_normal(co) * 0.1,
            "norm.weight": 1 + 0.1 * r.standard_normal(co), "norm.bias": 0.1 * r.standard_normal(co)}
    for h in range(4):
        P[f"output_heads.{h}"] = {"weight": r.standard_normal((2, 2, 1)),
                                  "bias": r.standard_normal(2) * 0.1}
    P32 = {k: {kk: vv.astype(np.float32) for kk, vv in v.items()} for k, v in P.items()}
    return cfg, P32


def build(dev, cfg, P):
    sep = nn.Separator(dev, cfg["input_channels"], cfg["num_stems"], cfg["channels"],
                       cfg["kernel_size"], cfg["stride"], cfg["num_groups"])
    sep.load_state(P)
    return sep


@pytest.mark.parametrize("n", [4000, 4096, 777])
def test_separate_one_pass(dev, stream, n):
    cfg, P = model()
    say(f"separate one pass n={n}")
    x = RNG.uniform(-1, 1, 2 * n).astype(np.float32)
    sep = build(dev, cfg, P)
    out = sep.separate(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(60000)
    ref = osep.separate_time(x, P, cfg)
    assert out.shape == ref.shape == (4, 2 * n)
    assert_close(out.to_numpy(), ref, 1e-4, 1e-3, "separate")


@pytest.mark.parametrize("n,seg,ovl", [(10000, 3000, 500), (10000, 3000, 0), (9000, 4000, 3999),
                                       (5000, 5000, 100), (6000, 2500, 2000)])
def test_separate_long(dev, stream, n, seg, ovl):
    cfg, P = model()
    say(f"separate long n={n} segment={seg} overlap={ovl}")
    x = RNG.uniform(-1, 1, 2 * n).astype(np.float32)
    sep = build(dev, cfg, P)
    out = sep.separate_long(nn.Tensor.from_numpy(dev, x), seg, ovl, stream)
    stream.sync(60000)
    ref = osep.separate_long(x, 2, seg, ovl, lambda s: osep.separate_time(s, P, cfg))
    assert_close(out.to_numpy(), ref, 1e-4, 1e-3, "separate_long")


def test_separator_errors(dev, stream):
    cfg, P = model(levels=2)
    sep = build(dev, cfg, P)
    with pytest.raises(nn.MNNError):
        sep.load("time_encoder.7.conv.weight", np.zeros(3, np.float32))
    with pytest.raises(nn.MNNError):
        sep.load("unknown.weight", np.zeros(3, np.float32))
    with pytest.raises(nn.MNNError):
        sep.load("time_encoder.0.conv.weight", np.zeros(3, np.float32))  # wrong size
    x = nn.Tensor.from_numpy(dev, np.zeros(2 * 100 + 1, np.float32))  # not a whole frame count
    with pytest.raises(nn.MNNError):
        sep.separate(x, stream)
    x = nn.Tensor.from_numpy(dev, np.zeros(2 * 1000, np.float32))
    with pytest.raises(nn.MNNError):
        sep.separate_long(x, 300, 300, stream)  # overlap must be below the segment


def test_separator_weights_from_demucs_named_safetensors(dev, stream, tmp_path):
    """HTDemucs.loadWeights(from:) with a Demucs-named file: names mapped by the detected
    convention (tencoder.i.norm1 -> time_encoder.i.norm, tdecoder.j.conv_tr ->
    time_decoder.j.conv_transpose, ...), frequency-branch tensors skipped, then the separation
    matches the oracle on the same weights."""
    from safetensors.numpy import save_file
    cfg, P = model(levels=2)
    say("separator weights from a Demucs-named safetensors file")
    flat = {}
    for k, v in P.items():
        for kk, vv in v.items():
            name = f"{k}.{kk}"
            name = (name.replace("time_encoder.", "tencoder.").replace(".norm.", ".norm1.")
                    if name.startswith("time_encoder.") else name)
            if name.startswith("time_decoder."):
                name = (name.replace("time_decoder.", "tdecoder.")
                        .replace(".conv_transpose.", ".conv_tr.").replace(".norm.", ".norm2."))
            flat[name] = np.ascontiguousarray(vv)
    flat["encoder.0.conv.weight"] = np.zeros((4, 2, 3, 3), np.float32)  # frequency branch
    flat["crosstransformer.layers.0.norm1.weight"] = np.ones(8, np.float32)
    save_file(flat, str(tmp_path / "demucs.safetensors"))
    st = nn.SafeTensors(tmp_path / "demucs.safetensors")
    assert st.create_weight_mapper().convention == "demucs"
    sep = nn.Separator(dev, 2, 4, cfg["channels"], 8, 4, 4)
    n_loaded = sep.load_safetensors(st)
    assert n_loaded == sum(len(v) for v in P.values())
    x = RNG.uniform(-1, 1, 2 * 3000).astype(np.float32)
    out = sep.separate(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(60000)
    assert_close(out.to_numpy(), osep.separate_time(x, P, cfg), 1e-4, 1e-3, "separate")


def _flat(P, head_prefix):
    flat = {}
    for k, v in P.items():
        if k.startswith("output_heads."):
            k = head_prefix + k[len("output_heads."):]
        for kk, vv in v.items():
            flat[f"{k}.{kk}"] = np.ascontiguousarray(vv)
    return flat


def test_separator_weights_with_reference_head_names(dev, stream, tmp_path):
    """A MetalAudio-named file as HTDemucs.loadWeights reads it: output heads under
    'time_output_heads.{i}' (HTDemucs.swift:1021). The heads must load (not stay zero), so the
    stems match the oracle."""
    from safetensors.numpy import save_file
    cfg, P = model(levels=2)
    say("separator weights, reference head names")
    save_file(_flat(P, "time_output_heads."), str(tmp_path / "ma.safetensors"))
    st = nn.SafeTensors(tmp_path / "ma.safetensors")
    assert st.create_weight_mapper().convention == "metalaudio"
    sep = nn.Separator(dev, 2, 4, cfg["channels"], 8, 4, 4)
    assert sep.load_safetensors(st) == sum(len(v) for v in P.values())
    x = RNG.uniform(-1, 1, 2 * 2000).astype(np.float32)
    out = sep.separate(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(60000)
    ref = osep.separate_time(x, P, cfg)
    assert np.abs(ref).max() > 0.1
    assert_close(out.to_numpy(), ref, 1e-4, 1e-3, "separate, reference head names")
    # the same names through the per-tensor loader
    sep2 = nn.Separator(dev, 2, 4, cfg["channels"], 8, 4, 4)
    for name, v in _flat(P, "time_output_heads.").items():
        sep2.load(name, v)
    out2 = sep2.separate(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(60000)
    assert_close(out2.to_numpy(), ref, 1e-4, 1e-3, "separate, per-tensor reference names")


@pytest.mark.parametrize("drop", ["time_encoder.1.conv.weight", "time_encoder.0.norm.bias",
                                  "time_decoder.0.conv_transpose.weight",
                                  "time_decoder.1.norm.weight"])
def test_separator_file_missing_required_tensor(dev, tmp_path, drop):
    """HTDemucs.loadWeights throws tensorNotFound for every encoder / decoder conv and norm tensor
    (HTDemucs.swift:892-937): a file without one is rejected and loads nothing."""
    from safetensors.numpy import save_file
    cfg, P = model(levels=2)
    say(f"separator file without {drop}")
    flat = _flat(P, "time_output_heads.")
    del flat[drop]
    save_file(flat, str(tmp_path / "m.safetensors"))
    st = nn.SafeTensors(tmp_path / "m.safetensors")
    sep = nn.Separator(dev, 2, 4, cfg["channels"], 8, 4, 4)
    with pytest.raises(nn.MNNError) as e:
        sep.load_safetensors(st)
    assert e.value.name == "MNN_ERR_TENSOR_NOT_FOUND" and drop in str(e.value)


def test_separator_file_without_optional_tensors(dev, stream, tmp_path):
    """Conv biases and output heads are optional (loadConv1DWeights, SafeTensorsLoader.swift:
    238-258; HTDemucs.swift:1017-1029): without them the biases stay zero and the file loads."""
    from safetensors.numpy import save_file
    cfg, P = model(levels=2)
    say("separator file without conv biases")
    flat = {k: v for k, v in _flat(P, "time_output_heads.").items()
            if not (k.endswith("conv.bias") or k.endswith("conv_transpose.bias"))}
    save_file(flat, str(tmp_path / "nb.safetensors"))
    sep = nn.Separator(dev, 2, 4, cfg["channels"], 8, 4, 4)
    assert sep.load_safetensors(nn.SafeTensors(tmp_path / "nb.safetensors")) == len(flat)
    P0 = {k: {kk: (np.zeros_like(vv) if kk in ("conv.bias", "conv_transpose.bias") else vv)
              for kk, vv in v.items()} for k, v in P.items()}
    x = RNG.uniform(-1, 1, 2 * 1500).astype(np.float32)
    out = sep.separate(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(60000)
    assert_close(out.to_numpy(), osep.separate_time(x, P0, cfg), 1e-4, 1e-3, "zero conv biases")
