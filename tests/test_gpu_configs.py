"""Full-size parity of the five benchmark configurations against the fp64 oracle.

fp32 bar: |gpu - oracle| <= 1e-4 + 1e-3 * |oracle| per element (the path's stated tolerance).
Inputs and weights are the seeded synthetic workloads that bench.py times.
"""
import sys

import numpy as np
import pytest

import oracle
from metalaudio_amd import nn, workloads
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu
ATOL, RTOL = 1e-4, 1e-3


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    return nn.AudioDevice(0)


@pytest.fixture(scope="module")
def stream(dev):
    return nn.Stream(dev)


def test_config1_conv_gn_gelu(dev, stream):
    say("config 1: Conv1D 2->48 k8 s4 -> GroupNorm(1) -> GELU on 44100 samples")
    c = workloads.config1()
    conv = nn.Conv1D(dev, 2, 48, 8, stride=4, padding=0, input_length=44100)
    conv.load_weights(c["conv_w"], c["conv_b"])
    gn = nn.GroupNorm(dev, 1, 48)
    gn.load_parameters(c["gn_w"], c["gn_b"])
    gelu = nn.GELU(dev, [1, 48, 11024])
    seq = nn.Sequential(dev)
    for l in (conv, gn, gelu):
        seq.add_unchecked(l)
    seq.build()
    out = seq.forward(nn.Tensor.from_numpy(dev, c["x"]), stream)
    stream.sync(60000)
    got = out.to_numpy().reshape(1, 48, 11024)
    y = oracle.conv1d(c["x"], c["conv_w"], c["conv_b"], stride=4, padding=0)
    ref = oracle.gelu_layer(oracle.group_norm(y, 1, c["gn_w"], c["gn_b"]))
    assert_close(got, ref, ATOL, RTOL, "config 1")


def test_config2_linear_layernorm(dev, stream):
    say("config 2: Linear 512->2048 on [2048, 512] + LayerNorm(2048), fp32")
    c = workloads.config2()
    lin = nn.Linear(dev, 512, 2048)
    lin.load_weights(c["w"], c["b"])
    ln = nn.LayerNorm(dev, 2048)
    ln.load_parameters(c["ln_w"], c["ln_b"])
    x = nn.Tensor.from_numpy(dev, c["x"])
    y = lin(x, stream)
    z = ln(y, stream)
    stream.sync(60000)
    ref_y = oracle.linear(c["x"], c["w"], c["b"])
    assert_close(y.to_numpy(), ref_y, ATOL, RTOL, "config 2 linear")
    assert_close(z.to_numpy(), oracle.layer_norm(ref_y, c["ln_w"], c["ln_b"]), ATOL, RTOL,
                 "config 2 layernorm")


def test_config3_transformer_layer(dev, stream):
    say("config 3: pre-norm MHSA + FFN, seq 2048, E 512, H 8")
    c = workloads.config3()
    t = nn.TransformerLayer(dev, c["embed"], c["heads"], c["ffn"])
    t.load_state(c["params"])
    x = nn.Tensor.from_numpy(dev, c["x"])
    out = t(x, stream)
    stream.sync(60000)
    ref = oracle.transformer_layer(c["x"], c["params"], c["heads"])
    assert_close(out.to_numpy(), ref, ATOL, RTOL, "config 3")


def _encoder(dev, c, precision="f32"):
    seq = nn.Sequential(dev)
    blocks = []
    for cin, cout, lv in zip(workloads.ENC_CHANNELS[:-1], workloads.ENC_CHANNELS[1:], c["levels"]):
        b = nn.UNetEncoderBlock(dev, cin, cout, 8, 4, 1, rewrite=True, precision=precision)
        b.load_weights(lv["conv.weight"], lv["conv.bias"], lv["norm.weight"], lv["norm.bias"],
                       lv["rewrite.weight"], lv["rewrite.bias"])
        blocks.append(b)
        seq.add(b)
    seq.build()
    return seq, blocks


@pytest.mark.parametrize("stress", [False, True])
def test_config4_time_encoder(dev, stream, stress):
    say(f"config 4: 4-level time encoder on 343980 samples (stress={stress})")
    c = workloads.config4(stress=stress)
    seq, _blocks = _encoder(dev, c)
    out = seq.forward(nn.Tensor.from_numpy(dev, c["x"]), stream)
    stream.sync(60000)
    got = out.to_numpy()
    assert got.shape == (1, 384, 1344)
    ref = oracle.time_encoder(c["x"], c["levels"])
    assert_close(got, ref, ATOL, RTOL, "config 4")


@pytest.mark.parametrize("batch", [1, 4])
def test_config5_cross_transformer(dev, stream, batch):
    say(f"config 5: cross transformer, 5 layers, time 1344 / freq 2688, batch {batch}")
    c = workloads.config5(batch=batch)
    ct = nn.CrossTransformerEncoder(dev, c["embed"], c["heads"], c["ffn"], c["layers"],
                                    c["layer_scale"])
    ct.load_state(c["params"])
    tt, ft = nn.Tensor.from_numpy(dev, c["time"]), nn.Tensor.from_numpy(dev, c["freq"])
    to, fo = nn.Tensor(dev, tt.shape), nn.Tensor(dev, ft.shape)
    ct.forward_cross(tt, ft, to, fo, stream)
    stream.sync(60000)
    rt, rf = oracle.cross_transformer(c["time"], c["freq"], c["params"], c["layers"], c["heads"])
    assert_close(to.to_numpy(), rt, ATOL, RTOL, "config 5 time")
    assert_close(fo.to_numpy(), rf, ATOL, RTOL, "config 5 freq")
    # the update itself (output - input, scaled by 1e-4) must also match to fp32 accuracy
    for got, ref, x, name in ((to.to_numpy(), rt, c["time"], "time"),
                              (fo.to_numpy(), rf, c["freq"], "freq")):
        du = (got.astype(np.float64) - x) / 1e-4
        rdu = (ref - x) / 1e-4
        assert_close(du, rdu, 2e-2, 2e-2, f"config 5 {name} update / LayerScale")


def test_config5_in_place_and_repeatable(dev, stream):
    say("config 5: in-place outputs and bitwise repeatability")
    c = workloads.config5(batch=1, time_len=400, freq_len=800)
    ct = nn.CrossTransformerEncoder(dev, c["embed"], c["heads"], c["ffn"], c["layers"],
                                    c["layer_scale"])
    ct.load_state(c["params"])
    tt, ft = nn.Tensor.from_numpy(dev, c["time"]), nn.Tensor.from_numpy(dev, c["freq"])
    to, fo = nn.Tensor(dev, tt.shape), nn.Tensor(dev, ft.shape)
    ct.forward_cross(tt, ft, to, fo, stream)
    a = to.to_numpy(stream), fo.to_numpy(stream)
    ct.forward_cross(tt, ft, to, fo, stream)
    b = to.to_numpy(stream), fo.to_numpy(stream)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    ct.forward_cross(tt, ft, tt, ft, stream)  # outputs alias inputs
    np.testing.assert_array_equal(tt.to_numpy(stream), a[0])
    np.testing.assert_array_equal(ft.to_numpy(stream), a[1])


# ----------------------------------------------------------------------------- hd = 48 attention
# The configuration-5 attention (E 384, H 8, head dim 48, batch 4) at its real lengths, per
# element at the fp32 bar. The projections use std 0.1 (in) / 0.05 (out) rather than the
# benchmark's 0.02 so that the scores spread over several units (a peaked softmax) and the
# outputs are O(1): an error in the kernel's key blocks, its online rescale or its query tiling
# then moves outputs by far more than 1e-4 + 1e-3 |ref|.
ATTN5_CASES = [(1344, 1344, False), (2688, 2688, False), (1344, 2688, True), (2688, 1344, True),
               # few query workgroups: the keys split into 4 ranges merged by the combine step
               (64, 2688, True), (300, 1344, True)]


@pytest.mark.parametrize("sq,sk,cross", ATTN5_CASES,
                         ids=[f"{'cross' if c else 'self'}-{q}x{k}" for q, k, c in ATTN5_CASES])
def test_mha_config5_lengths(dev, stream, sq, sk, cross):
    say(f"mha hd 48, batch 4, Sq {sq} Sk {sk} {'cross' if cross else 'self'}")
    E, H, B = 384, 8, 4
    r = np.random.Generator(np.random.PCG64(5100 + sq + 3 * sk + int(cross)))
    w_in = (r.standard_normal((3 * E, E)) * 0.1).astype(np.float32)
    b_in = (r.standard_normal(3 * E) * 0.05).astype(np.float32)
    w_out = (r.standard_normal((E, E)) * 0.05).astype(np.float32)
    b_out = (r.standard_normal(E) * 0.05).astype(np.float32)
    q = r.standard_normal((B, sq, E)).astype(np.float32)
    kv = r.standard_normal((B, sk, E)).astype(np.float32) if cross else None
    layer = nn.MultiHeadAttention(dev, E, H)
    layer.load_weights(w_in, b_in, w_out, b_out)
    qt = nn.Tensor.from_numpy(dev, q)
    out = nn.Tensor(dev, q.shape)
    if cross:
        layer.forward_cross(qt, nn.Tensor.from_numpy(dev, kv), out, stream)
    else:
        layer.forward(qt, out, stream)
    stream.sync(60000)
    ref = oracle.mha(q, kv, w_in, b_in, w_out, b_out, H)
    assert float(np.abs(ref).mean()) > 0.1  # O(1) outputs: the tolerance is a real bound
    assert_close(out.to_numpy(), ref, ATOL, RTOL, "mha config-5 lengths")


def test_config5_full_lengths_layerscale_one(dev, stream):
    """Configuration-5 shapes (batch 4, time 1344 / freq 2688) through one self-attention layer
    and one cross-attention layer with LayerScale 1, so each sub-block's update enters the output
    at full strength and is checked per element at the fp32 bar."""
    say("config 5 shapes, 2 layers (self, cross), LayerScale 1, batch 4")
    c = workloads.config5(stress=True, layers=2)
    p = {}
    for k, v in c["params"].items():
        if "gamma_" in k:
            v = np.ones_like(v)
        elif "in_proj_weight" in k:
            v = v * 5.0  # std 0.1: peaked attention
        elif k.endswith(("out_proj_weight", "linear1.weight", "linear2.weight")):
            v = v * 2.5
        p[k] = v.astype(np.float32)
    ct = nn.CrossTransformerEncoder(dev, c["embed"], c["heads"], c["ffn"], 2, 1e-4)
    ct.load_state(p)
    tt, ft = nn.Tensor.from_numpy(dev, c["time"]), nn.Tensor.from_numpy(dev, c["freq"])
    to, fo = nn.Tensor(dev, tt.shape), nn.Tensor(dev, ft.shape)
    ct.forward_cross(tt, ft, to, fo, stream)
    stream.sync(60000)
    rt, rf = oracle.cross_transformer(c["time"], c["freq"], p, 2, c["heads"])
    for got, ref, x, name in ((to.to_numpy(), rt, c["time"], "time"),
                              (fo.to_numpy(), rf, c["freq"], "freq")):
        upd = np.abs(ref - x)
        assert float(upd.mean()) > 0.1, f"{name}: update too small to test ({upd.mean():.3e})"
        assert_close(got, ref, ATOL, RTOL, f"config 5 shapes, LayerScale 1, {name}")
