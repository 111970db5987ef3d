"""Pins the CPU oracle (oracle/layers.py) before it is trusted as the parity reference.

Each oracle function is checked against something that does not restate its formula:
  * the reference's committed golden vectors (time_encoder_level{0,1}, converted to npz),
  * closed-form known-answer tests taken from the reference's own test suite,
  * independent library routines (torch CPU: conv1d, group_norm, layer_norm, gelu, glu,
    linear, nn.MultiheadAttention, nn.TransformerEncoderLayer),
  * invariants (normalised mean 0 / variance 1, softmax rows, length formulas).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from metalaudio_amd import workloads
from tests.conftest import assert_close

torch.set_num_threads(4)
RNG = np.random.default_rng(7)


def t64(a):
    return torch.from_numpy(np.asarray(a, np.float64))


# ----------------------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("name", ["time_encoder_level0", "time_encoder_level1"])
def test_encoder_block_matches_reference_fixture(golden_dir, name):
    """HTDemucsValidationTests.swift:37-117 fixtures: per element abs <= 1e-4 or rel <= 1e-3."""
    d = np.load(golden_dir / f"{name}.npz")
    cin, cout, k, s, g = (int(v) for v in d["config"])
    y = oracle.encoder_block(d["input"], d["conv_weight"], d["conv_bias"], d["norm_weight"],
                             d["norm_bias"], g, kernel_size=k, stride=s)
    ref = d["output"].astype(np.float64)
    err = np.abs(y - ref)
    ok = (err <= 1e-4) | (err <= 1e-3 * np.abs(ref))
    assert ok.all(), f"max abs {err.max():.3e}"
    assert err.max() < 1e-5  # the fixture is fp32 torch output; the oracle is fp64


# ----------------------------------------------------------------------------- closed forms
def test_gelu_reference_table():
    """IntegrationTests.swift:28-67 (tanh-approximation table, accuracy 1e-3)."""
    x = np.array([-3.0, -2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0, 3.0, 5.0])
    expected = np.array([-0.00364, -0.04550, -0.1588, -0.1543, 0.0, 0.3457, 0.8412, 1.9546,
                         2.9964, 5.0000])
    assert np.all(np.abs(oracle.gelu_layer(x) - expected) <= 1e-3)
    assert np.all(np.abs(oracle.gelu_tanh(x) - expected) <= 1e-3)


def test_gelu_clamp_semantics():
    """Activations.swift:124-137: x > 10 -> x, x < -10 -> 0."""
    x = np.array([-50.0, -10.5, 10.5, 50.0])
    np.testing.assert_array_equal(oracle.gelu_layer(x), [0.0, 0.0, 10.5, 50.0])


def test_gelu_matches_torch_tanh_gelu():
    x = RNG.standard_normal(10000) * 4
    ref = F.gelu(t64(x), approximate="tanh").numpy()
    # the reference literal 0.7978845608 differs from sqrt(2/pi) by 2.9e-12
    np.testing.assert_allclose(oracle.gelu_tanh(x), ref, rtol=0, atol=1e-10)


def test_layernorm_closed_form():
    """IntegrationTests.swift:336-374: [1,2,3,4] -> [-1.3416407, -0.4472136, 0.4472136, 1.3416407]."""
    y = oracle.layer_norm(np.array([1.0, 2.0, 3.0, 4.0]))
    np.testing.assert_allclose(y, [-1.3416407, -0.4472136, 0.4472136, 1.3416407], atol=1e-4)
    assert abs(y.mean()) < 1e-5 and abs(y.var() - 1.0) < 1e-4


def test_layernorm_matches_torch():
    x = RNG.standard_normal((37, 384)) * 3 + 1
    g, b = RNG.standard_normal(384), RNG.standard_normal(384)
    ref = F.layer_norm(t64(x), (384,), t64(g), t64(b), eps=1e-5).numpy()
    np.testing.assert_allclose(oracle.layer_norm(x, g, b), ref, rtol=1e-12, atol=1e-12)


def test_linear_closed_forms():
    """IntegrationTests.swift:259-324: W [[1,2,3],[4,5,6]], b [.1,.2], x [1,2,3] -> [14.1, 32.2];
    batch through identity-like weights."""
    w = np.array([[1, 2, 3], [4, 5, 6]], np.float64)
    np.testing.assert_allclose(oracle.linear(np.array([1.0, 2.0, 3.0]), w, [0.1, 0.2]),
                               [14.1, 32.2], atol=1e-12)
    wi = np.array([[1, 0, 0], [0, 1, 0]], np.float64)
    np.testing.assert_allclose(oracle.linear(np.array([[1, 2, 3], [4, 5, 6.0]]), wi),
                               [[1, 2], [4, 5]], atol=0)


@pytest.mark.parametrize("act", ["none", "relu", "leaky_relu", "gelu", "swish", "sigmoid", "tanh"])
def test_linear_matches_torch(act):
    x = RNG.standard_normal((13, 24))
    w, b = RNG.standard_normal((17, 24)), RNG.standard_normal(17)
    z = F.linear(t64(x), t64(w), t64(b))
    ref = {"none": z, "relu": F.relu(z), "leaky_relu": F.leaky_relu(z, 0.01),
           "gelu": F.gelu(z, approximate="tanh"), "swish": F.silu(z), "sigmoid": torch.sigmoid(z),
           "tanh": torch.tanh(z)}[act].numpy()
    np.testing.assert_allclose(oracle.linear(x, w, b, act=act), ref, rtol=1e-9, atol=1e-9)


def test_conv_identity_and_averaging():
    """Conv1DTests.swift:66-146 (padding 1, k 3)."""
    y = oracle.conv1d(np.array([[1.0, 2, 3, 4, 5]]), np.array([[[0.0, 1, 0]]]), padding=1)
    np.testing.assert_allclose(y, [[1, 2, 3, 4, 5]], atol=1e-12)
    w = np.full((1, 1, 3), 1.0 / 3.0)
    y = oracle.conv1d(np.array([[3.0] * 5]), w, padding=1)
    np.testing.assert_allclose(y, [[2, 3, 3, 3, 2]], atol=1e-12)


def test_conv_output_lengths():
    """DynamicConv1DTests.swift:373-390 (441000 -> 110250, reflect 3) and the config chains."""
    def lout(L, k=8, s=4, p=3):
        return (L + 2 * p - k) // s + 1
    assert lout(441000) == 110250
    L, chain = workloads.CHUNK_SAMPLES, []
    for _ in range(4):
        L = lout(L)
        chain.append(L)
    assert chain == [85995, 21499, 5375, 1344]
    assert lout(44100, p=0) == 11024


@pytest.mark.parametrize("cin,cout,k,s,p,d,g,mode", [
    (2, 48, 8, 4, 0, 1, 1, "zeros"),
    (2, 48, 8, 4, 3, 1, 1, "reflect"),
    (6, 12, 5, 2, 2, 2, 3, "zeros"),
    (48, 96, 8, 4, 3, 1, 1, "reflect"),
    (8, 8, 1, 1, 0, 1, 1, "zeros"),
])
def test_conv_matches_torch(cin, cout, k, s, p, d, g, mode):
    x = RNG.standard_normal((2, cin, 257))
    w = RNG.standard_normal((cout, cin // g, k))
    b = RNG.standard_normal(cout)
    xt = t64(x)
    if mode == "reflect":
        xt = F.pad(xt, (p, p), mode="reflect")
        ref = F.conv1d(xt, t64(w), t64(b), stride=s, dilation=d, groups=g)
    else:
        ref = F.conv1d(xt, t64(w), t64(b), stride=s, padding=p, dilation=d, groups=g)
    y = oracle.conv1d(x, w, b, stride=s, padding=p, dilation=d, groups=g, mode=mode)
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-10, atol=1e-10)


def test_round_bf16_matches_torch():
    x = np.concatenate([RNG.standard_normal(20000) * 10, [0.0, -0.0, 1e-40, 3.4e38, -2.5]])
    x = x.astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(oracle.round_bf16(x), ref)


def test_reflect_pad_matches_torch():
    x = RNG.standard_normal((3, 11))
    ref = F.pad(t64(x)[None], (3, 3), mode="reflect")[0].numpy()
    np.testing.assert_array_equal(oracle.reflect_pad(x, 3), ref)


@pytest.mark.parametrize("groups", [1, 8])
def test_group_norm_matches_torch_and_invariants(groups):
    x = RNG.standard_normal((2, 48, 301)) * 2 + 0.5
    g, b = RNG.standard_normal(48), RNG.standard_normal(48)
    ref = F.group_norm(t64(x), groups, t64(g), t64(b), eps=1e-5).numpy()
    np.testing.assert_allclose(oracle.group_norm(x, groups, g, b), ref, rtol=1e-10, atol=1e-10)
    y = oracle.group_norm(x, groups).reshape(2, groups, -1)   # GroupNormTests.swift:478-533
    assert np.all(np.abs(y.mean(-1)) < 1e-10) and np.all(np.abs(y.var(-1) - 1) < 1e-3)


def test_glu_matches_torch_and_sigmoid_extremes():
    x = RNG.standard_normal((2, 20, 33)) * 5
    np.testing.assert_allclose(oracle.glu(x, axis=-2), F.glu(t64(x), dim=-2).numpy(), rtol=1e-12,
                               atol=1e-14)
    s = oracle.stable_sigmoid(np.array([-1000.0, -88.0, 0.0, 88.0, 1000.0]))
    assert s[0] == s[1] and s[3] == s[4] and s[2] == 0.5 and np.all(np.isfinite(s))


def _torch_mha(E, H, w_in, b_in, w_out, b_out):
    m = torch.nn.MultiheadAttention(E, H, bias=True, batch_first=True, dtype=torch.float64)
    with torch.no_grad():
        m.in_proj_weight.copy_(t64(w_in))
        m.in_proj_bias.copy_(t64(b_in))
        m.out_proj.weight.copy_(t64(w_out))
        m.out_proj.bias.copy_(t64(b_out))
    return m.eval()


@pytest.mark.parametrize("E,H,Sq,Sk,cross", [(64, 4, 19, 19, False), (96, 2, 17, 29, True),
                                             (384, 8, 33, 65, True)])
def test_mha_matches_torch(E, H, Sq, Sk, cross):
    """Packed in_proj rows Q;K;V and out_proj as nn.MultiheadAttention (Attention.swift:10-14)."""
    w_in, b_in = RNG.standard_normal((3 * E, E)) * 0.1, RNG.standard_normal(3 * E) * 0.1
    w_out, b_out = RNG.standard_normal((E, E)) * 0.1, RNG.standard_normal(E) * 0.1
    q = RNG.standard_normal((2, Sq, E))
    kv = RNG.standard_normal((2, Sk, E)) if cross else q
    m = _torch_mha(E, H, w_in, b_in, w_out, b_out)
    with torch.no_grad():
        ref = m(t64(q), t64(kv), t64(kv), need_weights=False)[0].numpy()
    got = oracle.mha(q, kv if cross else None, w_in, b_in, w_out, b_out, H)
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-8)


def test_mha_scale_and_identity_weights():
    """AttentionTests.swift:505-519 (scale 1/sqrt(hd)) and :586-642 (identity weights bounded):
    with identity projections and one key, the output equals the value row."""
    E, H = 8, 2
    w_in = np.concatenate([np.eye(E)] * 3)
    x = RNG.standard_normal((1, E))
    y = oracle.mha(x, None, w_in, np.zeros(3 * E), np.eye(E), np.zeros(E), H)
    np.testing.assert_allclose(y, x, atol=1e-9)
    xs = RNG.standard_normal((5, E))
    y = oracle.mha(xs, None, w_in, None, np.eye(E), None, H)
    assert np.all(np.abs(y) <= np.abs(xs).max(0) + 1e-12)


def test_feed_forward_matches_torch():
    x = RNG.standard_normal((9, 32))
    w1, b1 = RNG.standard_normal((64, 32)), RNG.standard_normal(64)
    w2, b2 = RNG.standard_normal((32, 64)), RNG.standard_normal(32)
    ref = F.linear(F.gelu(F.linear(t64(x), t64(w1), t64(b1)), approximate="tanh"), t64(w2), t64(b2))
    np.testing.assert_allclose(oracle.feed_forward(x, w1, b1, w2, b2), ref.numpy(), rtol=1e-10,
                               atol=1e-10)


def test_transformer_layer_matches_torch_encoder_layer():
    """Config-3 layer (pre-norm, no LayerScale) against nn.TransformerEncoderLayer(norm_first)."""
    cfg = workloads.config3(stress=True, seq=40)
    E, H, Hd, p = cfg["embed"], cfg["heads"], cfg["ffn"], cfg["params"]
    m = torch.nn.TransformerEncoderLayer(E, H, Hd, dropout=0.0, batch_first=True, norm_first=True,
                                         activation=lambda z: F.gelu(z, approximate="tanh"),
                                         dtype=torch.float64).eval()
    with torch.no_grad():
        m.self_attn.in_proj_weight.copy_(t64(p["attn.in_proj_weight"]))
        m.self_attn.in_proj_bias.copy_(t64(p["attn.in_proj_bias"]))
        m.self_attn.out_proj.weight.copy_(t64(p["attn.out_proj_weight"]))
        m.self_attn.out_proj.bias.copy_(t64(p["attn.out_proj_bias"]))
        for n in ("linear1", "linear2"):
            getattr(m, n).weight.copy_(t64(p[n + ".weight"]))
            getattr(m, n).bias.copy_(t64(p[n + ".bias"]))
        for n in ("norm1", "norm2"):
            getattr(m, n).weight.copy_(t64(p[n + ".weight"]))
            getattr(m, n).bias.copy_(t64(p[n + ".bias"]))
        ref = m(t64(cfg["x"])[None])[0].numpy()
    np.testing.assert_allclose(oracle.transformer_layer(cfg["x"], p, H), ref, rtol=1e-9,
                               atol=1e-9)


def _metalnn_encoder_torch(cfg, plant=None):
    """The reference CrossTransformerEncoder's layer loop (Transformer.swift:626-667) with
    TransformerLayer.forward (:441-498) composed from torch library routines: F.layer_norm,
    torch's MultiheadAttention with the packed in_proj, Linear -> tanh GELU -> Linear, and one
    addResidual per sub-block, in the order of :467-495. `plant` names a mistake planted in this
    checker ("double_time_self": the time self-attention residual added twice;
    "cross_reads_updated_time": the freq cross-attention's keys / values normalised from the time
    state after its own cross update instead of the timeNormed of :478)."""
    p, E, H = cfg["params"], cfg["embed"], cfg["heads"]

    def ln(x, pre):
        return F.layer_norm(x, (E,), t64(p[pre + ".weight"]), t64(p[pre + ".bias"]), 1e-5)

    def attn(q, kv, pre):
        m = _torch_mha(E, H, p[pre + ".in_proj_weight"], p[pre + ".in_proj_bias"],
                       p[pre + ".out_proj.weight"], p[pre + ".out_proj.bias"])
        return m(q, kv, kv, need_weights=False)[0]

    def ffn(x, pre):
        h = F.gelu(F.linear(x, t64(p[pre + ".linear1.weight"]), t64(p[pre + ".linear1.bias"])),
                   approximate="tanh")
        return F.linear(h, t64(p[pre + ".linear2.weight"]), t64(p[pre + ".linear2.bias"]))

    with torch.no_grad():
        T, Fr = t64(cfg["time"]), t64(cfg["freq"])
        for i in range(cfg["layers"]):
            L = f"layers.{i}."
            h = ln(T, L + "norm_time_self")                      # :468
            a = attn(h, h, L + "self_attn_time")                 # :469
            T = T + a                                            # :470
            if plant == "double_time_self":
                T = T + a
            h = ln(Fr, L + "norm_freq_self")                     # :473-475
            Fr = Fr + attn(h, h, L + "self_attn_freq")
            tn, fn = ln(T, L + "norm_time_cross"), ln(Fr, L + "norm_freq_cross")  # :478-479
            T = T + attn(tn, fn, L + "cross_attn_time")          # :480-481
            if plant == "cross_reads_updated_time":
                tn = ln(T, L + "norm_time_cross")
            Fr = Fr + attn(fn, tn, L + "cross_attn_freq")        # :484-485
            T = T + ffn(ln(T, L + "norm_time_ffn"), L + "ffn_time")      # :488-490
            Fr = Fr + ffn(ln(Fr, L + "norm_freq_ffn"), L + "ffn_freq")   # :493-495
    return T.numpy(), Fr.numpy()


def test_cross_transformer_metalnn_matches_torch_composition():
    """The reference-structured encoder against torch library routines composed in the order of
    Transformer.swift:467-495 (one residual per sub-block)."""
    cfg = workloads.cross_encoder_metalnn(batch=2, time_len=13, freq_len=21, embed=16, heads=4,
                                          ffn=32, layers=2)
    T, Fq = oracle.cross_transformer_metalnn(cfg["time"], cfg["freq"], cfg["params"],
                                             cfg["layers"], cfg["heads"])
    Tt, Ft = _metalnn_encoder_torch(cfg)
    np.testing.assert_allclose(T, Tt, rtol=1e-9, atol=1e-9)  # both fp64
    np.testing.assert_allclose(Fq, Ft, rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("plant", ["double_time_self", "cross_reads_updated_time"])
def test_cross_transformer_metalnn_planted_mistakes_fail(plant):
    """A mistake planted in the checker moves its result well outside the oracle's agreement
    (1e-9), so the composition above pins the residual count and the cross-attention inputs."""
    cfg = workloads.cross_encoder_metalnn(batch=2, time_len=13, freq_len=21, embed=16, heads=4,
                                          ffn=32, layers=2)
    T, Fq = oracle.cross_transformer_metalnn(cfg["time"], cfg["freq"], cfg["params"],
                                             cfg["layers"], cfg["heads"])
    Tp, Fp = _metalnn_encoder_torch(cfg, plant=plant)
    assert max(np.max(np.abs(Tp - T)), np.max(np.abs(Fp - Fq))) > 1e-3


def test_cross_transformer_metalnn_identity_when_updates_vanish():
    """Every sub-block adds to its branch: with the out-projections and the FFN's second linear
    zeroed, the encoder returns its inputs exactly."""
    cfg = workloads.cross_encoder_metalnn(batch=1, time_len=7, freq_len=9, embed=8, heads=2,
                                          ffn=16, layers=2)
    p = dict(cfg["params"])
    for k in p:
        if ".out_proj." in k or ".linear2." in k:
            p[k] = np.zeros_like(p[k])
    T, Fq = oracle.cross_transformer_metalnn(cfg["time"], cfg["freq"], p, 2, cfg["heads"])
    np.testing.assert_array_equal(T, cfg["time"].astype(np.float64))
    np.testing.assert_array_equal(Fq, cfg["freq"].astype(np.float64))


def test_cross_transformer_matches_torch_composition():
    """Config-5 structure composed from torch library routines with strong LayerScale."""
    cfg = workloads.config5(stress=True, batch=1, time_len=21, freq_len=37, layers=3)
    p = dict(cfg["params"])
    for k in p:
        if "gamma_" in k:
            p[k] = np.full_like(p[k], 0.7)
    E, H = cfg["embed"], cfg["heads"]

    def ln(x, pre):
        return F.layer_norm(x, (E,), t64(p[pre + ".weight"]), t64(p[pre + ".bias"]), 1e-5)

    def attn(q, kv, pre):
        m = _torch_mha(E, H, p[pre + "in_proj_weight"], p[pre + "in_proj_bias"],
                       p[pre + "out_proj_weight"], p[pre + "out_proj_bias"])
        return m(q, kv, kv, need_weights=False)[0]

    def ffn(x, pre):
        h = F.gelu(F.linear(x, t64(p[pre + "linear1.weight"]), t64(p[pre + "linear1.bias"])),
                   approximate="tanh")
        return F.linear(h, t64(p[pre + "linear2.weight"]), t64(p[pre + "linear2.bias"]))

    with torch.no_grad():
        T, Fr = t64(cfg["time"]), t64(cfg["freq"])
        for i in range(3):
            a, b = f"layers.{i}.time.", f"layers.{i}.freq."
            if i % 2 == 0:
                outs = []
                for X, pre in ((T, a), (Fr, b)):
                    h = ln(X, pre + "norm1")
                    X = X + t64(p[pre + "gamma_1.scale"]) * attn(h, h, pre + "attn.")
                    X = X + t64(p[pre + "gamma_2.scale"]) * ffn(ln(X, pre + "norm2"), pre)
                    outs.append(X)
                T, Fr = outs
            else:
                Tn = T + t64(p[a + "gamma_1.scale"]) * attn(ln(T, a + "norm1"),
                                                            ln(Fr, a + "norm2"), a + "attn.")
                Fn = Fr + t64(p[b + "gamma_1.scale"]) * attn(ln(Fr, b + "norm1"),
                                                             ln(T, b + "norm2"), b + "attn.")
                Tn = Tn + t64(p[a + "gamma_2.scale"]) * ffn(ln(Tn, a + "norm3"), a)
                Fn = Fn + t64(p[b + "gamma_2.scale"]) * ffn(ln(Fn, b + "norm3"), b)
                T, Fr = Tn, Fn
    ot, of = oracle.cross_transformer(cfg["time"], cfg["freq"], p, 3, H)
    np.testing.assert_allclose(ot, T.numpy(), rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(of, Fr.numpy(), rtol=1e-9, atol=1e-9)


def test_time_encoder_matches_torch_composition():
    cfg = workloads.config4(stress=True, samples=4000)
    with torch.no_grad():
        y = t64(cfg["x"])
        for lv in cfg["levels"]:
            y = F.conv1d(F.pad(y, (3, 3), mode="reflect"), t64(lv["conv.weight"]),
                         t64(lv["conv.bias"]), stride=4)
            y = F.gelu(F.group_norm(y, 1, t64(lv["norm.weight"]), t64(lv["norm.bias"]), 1e-5),
                       approximate="tanh")
            y = F.glu(F.conv1d(y, t64(lv["rewrite.weight"]), t64(lv["rewrite.bias"])), dim=1)
    np.testing.assert_allclose(oracle.time_encoder(cfg["x"], cfg["levels"]), y.numpy(),
                               rtol=1e-9, atol=1e-10)


def test_planted_mistakes_are_caught(golden_dir):
    """Plausible oracle slips fail the golden fixture: GELU on the wrong side of GroupNorm,
    zero instead of reflect padding, and a transposed conv weight."""
    d = np.load(golden_dir / "time_encoder_level0.npz")
    ref = d["output"]
    y = oracle.conv1d(d["input"], d["conv_weight"], d["conv_bias"], stride=4, padding=3,
                      mode="reflect")
    wrong = oracle.group_norm(oracle.gelu_tanh(y), 8, d["norm_weight"], d["norm_bias"])
    assert np.abs(wrong - ref).max() > 1e-2
    yz = oracle.conv1d(d["input"], d["conv_weight"], d["conv_bias"], stride=4, padding=3,
                       mode="zeros")
    wrong = oracle.gelu_tanh(oracle.group_norm(yz, 8, d["norm_weight"], d["norm_bias"]))
    assert np.abs(wrong - ref).max() > 1e-3
    wt = d["conv_weight"][:, :, ::-1]
    wrong = oracle.encoder_block(d["input"], wt, d["conv_bias"], d["norm_weight"],
                                 d["norm_bias"], 8)
    assert np.abs(wrong - ref).max() > 1e-2


# ----------------------------------------------------------------------------- decoder path
@pytest.mark.parametrize("cin,cout,k,s,p,op,d,g", [
    (3, 4, 8, 4, 3, 2, 1, 1),    # the decoder block's transposed conv
    (6, 4, 5, 2, 1, 1, 2, 2),    # groups and dilation
    (4, 6, 3, 1, 0, 0, 1, 1),
    (2, 3, 4, 4, 0, 0, 1, 1),    # k == stride: no overlap between inputs
])
def test_conv_transpose1d_matches_gather_and_torch(cin, cout, k, s, p, op, d, g):
    """The scatter-form oracle against the reference kernel's per-output gather loop
    (DynamicConv1D.swift:588-640) and torch.nn.functional.conv_transpose1d."""
    x = RNG.standard_normal((cin, 11))
    w = RNG.standard_normal((cin, cout // g, k))
    b = RNG.standard_normal(cout)
    y = oracle.conv_transpose1d(x, w, b, s, p, op, d, g)
    np.testing.assert_allclose(y, oracle.conv_transpose1d_gather(x, w, b, s, p, op, d, g),
                               rtol=1e-12, atol=1e-12)
    ref = F.conv_transpose1d(t64(x)[None], t64(w), t64(b), s, p, op, g, d)[0]
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-12, atol=1e-12)
    assert y.shape[-1] == oracle.layers.conv_transpose1d_length(11, k, s, p, op, d)


def test_conv_transpose1d_closed_forms():
    """Nearest-neighbour upsampling (k == stride, ones) and a 1x1 transposed conv (W^T x)."""
    x = np.array([[1.0, -2.0, 3.0]])
    y = oracle.conv_transpose1d(x, np.ones((1, 1, 4)), stride=4)
    np.testing.assert_allclose(y, [[1, 1, 1, 1, -2, -2, -2, -2, 3, 3, 3, 3]])
    xm = RNG.standard_normal((3, 7))
    w = RNG.standard_normal((3, 5, 1))
    np.testing.assert_allclose(oracle.conv_transpose1d(xm, w), w[:, :, 0].T @ xm, atol=1e-12)


def test_decoder_block_shapes_and_composition():
    """UNetDecoderBlock: output length stride * L for k = 8, s = 4 (UNetTests.swift:405-440,
    upsampling); the block is concat -> conv_transpose1d -> GroupNorm -> GELU, checked against
    torch's ops."""
    cin, cskip, cout, L = 6, 6, 4, 13
    x, sk = RNG.standard_normal((2, cin, L)), RNG.standard_normal((2, cskip, L))
    w = RNG.standard_normal((cin + cskip, cout, 8)) * 0.3
    b, gm, bt = RNG.standard_normal(cout), 1 + RNG.standard_normal(cout) * 0.1, \
        RNG.standard_normal(cout) * 0.1
    y = oracle.decoder_block(x, sk, w, b, gm, bt, 2)
    assert y.shape == (2, cout, 4 * L)
    z = F.conv_transpose1d(torch.cat([t64(x), t64(sk)], 1), t64(w), t64(b), 4, 3, 2)
    ref = F.gelu(F.group_norm(z, 2, t64(gm), t64(bt), 1e-5), approximate="tanh")
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-10, atol=1e-10)
    # a skip given in the wrong order is not the same block
    wrong = oracle.decoder_block(sk, x, w, b, gm, bt, 2)
    assert np.abs(wrong - y).max() > 1e-2


@pytest.mark.parametrize("length,levels", [(1000, 1), (44_100, 5), (1024, 5), (343_980, 4),
                                           (1, 3), (257, 4)])
def test_unet_padding(length, levels):
    """UNetPaddingCalculatorTests (UNetTests.swift:635-690): the padded length is a multiple of
    stride**levels and the split is even with the odd sample on the right."""
    left, right, out = oracle.unet_padding(length, levels, 8, 4)
    assert out == length + left + right and out % 4 ** levels == 0
    assert out - length < 4 ** levels and right - left in (0, 1)
    if length % 4 ** levels == 0:
        assert left == right == 0
    assert oracle.unet_bottleneck_length(out, levels, 4) == out // 4 ** levels


def test_time_unet_lengths_round_trip():
    """A padded signal goes down 4 levels and back to its own length (HTDemucs.swift:521-548)."""
    _, _, L = oracle.unet_padding(3000, 2, 8, 4)
    ch = [2, 8, 16]
    enc, dec = [], []
    for i in range(2):
        enc.append({"conv.weight": RNG.standard_normal((ch[i + 1], ch[i], 8)) * 0.2,
                    "conv.bias": np.zeros(ch[i + 1]), "norm.weight": np.ones(ch[i + 1]),
                    "norm.bias": np.zeros(ch[i + 1])})
    for i in reversed(range(2)):
        dec.append({"conv_tr.weight": RNG.standard_normal((2 * ch[i + 1], ch[i], 8)) * 0.2,
                    "conv_tr.bias": np.zeros(ch[i]), "norm.weight": np.ones(ch[i]),
                    "norm.bias": np.zeros(ch[i]), "groups": min(8, ch[i])})
    y = oracle.time_unet(RNG.standard_normal((1, 2, L)), enc, dec)
    assert y.shape == (1, 2, L)


@pytest.mark.parametrize("act,alpha", [("relu", 0.01), ("leaky_relu", 0.01), ("leaky_relu", 0.3),
                                       ("gelu", 0.01), ("swish", 0.01), ("none", 0.01)])
def test_fused_conv1d_residual_vs_torch(act, alpha):
    """FusedConv1D.forwardWithResidual: act(conv + b) + residual (Conv1D.swift:1016-1023), against
    torch's conv1d and activations; a residual added before the activation (the plausible
    mistake) differs wherever the pre-activation is negative."""
    r = np.random.default_rng(61)
    x = r.standard_normal((2, 6, 50))
    w = r.standard_normal((8, 3, 5)) * 0.4
    b = r.standard_normal(8) * 0.3
    res = r.standard_normal((2, 8, 24)) * 2
    got = oracle.fused_conv1d(x, w, b, stride=2, padding=1, dilation=1, groups=2, act=act,
                              alpha=alpha, residual=res)
    y = F.conv1d(t64(x), t64(w), t64(b), stride=2, padding=1, groups=2)
    y = {"relu": F.relu, "leaky_relu": lambda v: F.leaky_relu(v, alpha),
         "gelu": lambda v: F.gelu(v, approximate="tanh"), "swish": F.silu,
         "none": lambda v: v}[act](y)
    np.testing.assert_allclose(got, (y + t64(res)).numpy(), rtol=1e-12, atol=1e-12)
    if act in ("relu", "leaky_relu"):
        before = oracle.activation(oracle.conv1d(x, w, b, stride=2, padding=1, groups=2) + res,
                                   act, alpha=alpha)
        assert np.abs(before - got).max() > 0.1


def test_torch_cpu_baseline_matches_oracle():
    """The torch-CPU restatement bench.py times as the CPU baseline computes the same function
    as the numpy oracle (config 4 on a short signal, config 5 at reduced lengths, stress
    parameters so that biases and affine terms are exercised)."""
    from oracle import torch_cpu as tc
    c4 = workloads.config4(stress=True, samples=6000)
    lv = [{k: tc.to_torch(v) for k, v in l.items()} for l in c4["levels"]]
    with torch.inference_mode():
        got = tc.time_encoder(tc.to_torch(c4["x"]), lv).numpy()
    assert_close(got, oracle.time_encoder(c4["x"], c4["levels"]), 1e-4, 1e-3, "torch encoder")
    c5 = workloads.config5(stress=True, batch=2, time_len=70, freq_len=130, layers=3)
    p = {k: (np.full_like(v, 0.5) if "gamma_" in k else v) for k, v in c5["params"].items()}
    pt = {k: tc.to_torch(v) for k, v in p.items()}
    with torch.inference_mode():
        t, f = tc.cross_transformer(tc.to_torch(c5["time"]), tc.to_torch(c5["freq"]), pt, 3, 8)
    rt, rf = oracle.cross_transformer(c5["time"], c5["freq"], p, 3, 8)
    assert_close(t.numpy(), rt, 1e-4, 1e-3, "torch transformer time")
    assert_close(f.numpy(), rf, 1e-4, 1e-3, "torch transformer freq")
