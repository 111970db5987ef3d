"""GPU parity of every hot-path layer against the fp64 oracle, through the C ABI.

fp32 bar (stated by the path's spec): |gpu - oracle| <= 1e-4 + 1e-3 * |oracle| per element.
"""
import ctypes
import sys

import numpy as np
import pytest

import oracle
from metalaudio_amd import _lib, nn
from metalaudio_amd import workloads
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu
ATOL, RTOL = 1e-4, 1e-3
RNG = np.random.default_rng(11)


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    d = nn.AudioDevice(0)
    yield d


@pytest.fixture(scope="module")
def stream(dev):
    s = nn.Stream(dev)
    yield s


def run_layer(layer, x, dev, stream):
    xt = nn.Tensor.from_numpy(dev, x)
    out = layer(xt, stream)
    stream.sync(60000)
    return out.to_numpy()


# ----------------------------------------------------------------------------- MFMA layouts
def _expected_raw(variant, a, b):
    """Expected raw registers under the lane layouts the kernels are written against."""
    lanes = np.arange(64)
    if variant in (0, 2):
        M = 32
        kper = 1 if variant == 0 else 8
        K = 2 * kper
        A = np.zeros((32, K))
        B = np.zeros((K, 32))
        for l in lanes:
            for t in range(kper):
                A[l % 32, kper * (l // 32) + t] = a[l * kper + t]
                B[kper * (l // 32) + t, l % 32] = b[l * kper + t]
        D = A @ B
        raw = np.zeros((64, 16))
        for l in lanes:
            for v in range(16):
                raw[l, v] = D[8 * (v // 4) + 4 * (l // 32) + v % 4, l % 32]
        return raw
    kper = 1 if variant == 1 else 8
    K = 4 * kper
    A = np.zeros((16, K))
    B = np.zeros((K, 16))
    for l in lanes:
        for t in range(kper):
            A[l % 16, kper * (l // 16) + t] = a[l * kper + t]
            B[kper * (l // 16) + t, l % 16] = b[l * kper + t]
    D = A @ B
    raw = np.zeros((64, 4))
    for l in lanes:
        for v in range(4):
            raw[l, v] = D[4 * (l // 16) + v, l % 16]
    return raw


@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_mfma_lane_layout(dev, variant):
    say(f"mfma probe variant {variant}")
    n = 64 if variant < 2 else 512
    # small integers / 4: exact in bf16 and in fp32 products and sums
    a = RNG.integers(-8, 9, n).astype(np.float32) / 4
    b = RNG.integers(-8, 9, n).astype(np.float32) / 4
    got = nn.mfma_probe(dev, variant, a, b)
    np.testing.assert_array_equal(got, _expected_raw(variant, a.astype(np.float64),
                                                      b.astype(np.float64)))


# ----------------------------------------------------------------------------- Conv1D
CONV_CASES = [
    # B, cin, cout, k, s, p, d, g, mode, act, L
    (1, 2, 48, 8, 4, 0, 1, 1, "explicit", "none", 44100),      # config 1 conv (direct)
    (1, 2, 48, 8, 4, 3, 1, 1, "reflect", "none", 4099),        # level-1 conv, ragged length
    (2, 48, 96, 8, 4, 3, 1, 1, "reflect", "none", 1031),       # implicit-GEMM MFMA, reflect
    (1, 96, 192, 8, 4, 3, 1, 1, "reflect", "gelu", 517),       # MFMA + fused GELU
    (1, 16, 32, 4, 1, 2, 1, 1, "explicit", "relu", 300),       # MFMA, zero padding
    (1, 6, 12, 5, 2, 2, 2, 3, "explicit", "swish", 203),       # groups + dilation (direct)
    (1, 1, 1, 3, 1, 1, 1, 1, "explicit", "none", 5),           # tiny
    (1, 8, 8, 3, 1, 0, 1, 1, "valid", "leaky_relu", 50),
    (1, 4, 16, 4, 2, 0, 1, 1, "same", "tanh", 33),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[str(c) for c in CONV_CASES])
def test_conv1d_parity(dev, stream, case):
    B, cin, cout, k, s, p, d, g, mode, act, L = case
    say(f"conv1d {case}")
    x = RNG.uniform(-1, 1, (B, cin, L)).astype(np.float32)
    w = (RNG.standard_normal((cout, cin // g, k)) * np.sqrt(2 / (cin // g * k))).astype(np.float32)
    b = (RNG.standard_normal(cout) * 0.1).astype(np.float32)
    layer = nn.DynamicConv1D(dev, cin, cout, k, s, padding_mode=mode, padding=p, dilation=d,
                             groups=g, activation=act)
    layer.load_weights(w, b)
    got = run_layer(layer, x, dev, stream)
    if mode == "same":
        eff = (k - 1) * d + 1
        lo = -(-L // s)
        p = max(0, (lo - 1) * s + eff - L) // 2
    elif mode == "valid":
        p = 0
    ref = oracle.conv1d(x, w, b, stride=s, padding=p, dilation=d, groups=g,
                        mode="reflect" if mode == "reflect" else "zeros")
    ref = oracle.activation(ref, act)
    assert_close(got, ref, ATOL, RTOL, f"conv {case}")


def test_conv1d_closed_forms(dev, stream):
    """Conv1DTests.swift:66-146: identity and averaging kernels, fixed-length Conv1D, padding 1."""
    say("conv closed forms")
    c = nn.Conv1D(dev, 1, 1, 3, padding=1, use_bias=False, input_length=5)
    c.load_weights([0, 1, 0])
    np.testing.assert_allclose(run_layer(c, np.array([[1, 2, 3, 4, 5.0]]), dev, stream),
                               [[1, 2, 3, 4, 5]], atol=1e-6)
    c.load_weights([1 / 3, 1 / 3, 1 / 3])
    np.testing.assert_allclose(run_layer(c, np.full((1, 5), 3.0), dev, stream),
                               [[2, 3, 3, 3, 2]], atol=1e-6)
    assert c.output_shape == (1, 5)


# ----------------------------------------------------------------------------- norms / activations
@pytest.mark.parametrize("B,C,L,G,act", [(1, 48, 11024, 1, "gelu"), (2, 48, 1000, 8, "none"),
                                         (1, 96, 4097, 3, "gelu"), (1, 4, 7, 2, "none")])
def test_groupnorm_parity(dev, stream, B, C, L, G, act):
    say(f"groupnorm {B, C, L, G, act}")
    x = (RNG.standard_normal((B, C, L)) * 3 + 0.7).astype(np.float32)
    gm = (1 + 0.2 * RNG.standard_normal(C)).astype(np.float32)
    bt = (0.2 * RNG.standard_normal(C)).astype(np.float32)
    layer = nn.GroupNorm(dev, G, C, activation=act)
    layer.load_parameters(gm, bt)
    got = run_layer(layer, x, dev, stream)
    ref = oracle.activation(oracle.group_norm(x, G, gm, bt), act)
    assert_close(got, ref, ATOL, RTOL, "groupnorm")


@pytest.mark.parametrize("rows,F", [(4, 4), (1000, 384), (333, 512), (2048, 2048), (17, 100),
                                    (3, 384), (257, 128), (10752, 384),
                                    # every width of the 16-lanes-per-row kernel (F = 64 * NV),
                                    # row counts that leave a partial last wave
                                    (65, 64), (130, 192), (7, 320), (1, 448)])
def test_layernorm_parity(dev, stream, rows, F):
    say(f"layernorm {rows}x{F}")
    x = (RNG.standard_normal((rows, F)) * 2 + 0.3).astype(np.float32)
    gm = (1 + 0.2 * RNG.standard_normal(F)).astype(np.float32)
    bt = (0.2 * RNG.standard_normal(F)).astype(np.float32)
    layer = nn.LayerNorm(dev, F)
    layer.load_parameters(gm, bt)
    got = run_layer(layer, x, dev, stream)
    assert_close(got, oracle.layer_norm(x, gm, bt), ATOL, RTOL, "layernorm")


def test_layernorm_closed_form(dev, stream):
    """IntegrationTests.swift:336-374."""
    say("layernorm closed form")
    got = run_layer(nn.LayerNorm(dev, 4), np.array([1.0, 2, 3, 4]), dev, stream)
    np.testing.assert_allclose(got, [-1.3416407, -0.4472136, 0.4472136, 1.3416407], atol=1e-4)


def test_gelu_parity_and_table(dev, stream):
    """IntegrationTests.swift:28-67 table at 1e-3, clamp semantics, and random values."""
    say("gelu")
    x = np.array([-3.0, -2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0, 3.0, 5.0], np.float32)
    got = run_layer(nn.GELU(dev, [10]), x, dev, stream)
    exp = [-0.00364, -0.04550, -0.1588, -0.1543, 0.0, 0.3457, 0.8412, 1.9546, 2.9964, 5.0]
    assert np.all(np.abs(got - exp) <= 1e-3)
    x = np.concatenate([RNG.standard_normal(100003) * 4, [-50, -10.5, 10.5, 50]]).astype(np.float32)
    got = run_layer(nn.GELU(dev, [x.size]), x, dev, stream)
    assert_close(got, oracle.gelu_layer(x), ATOL, RTOL, "gelu")
    assert got[-4] == 0.0 and got[-1] == 50.0


def test_glu_parity(dev, stream):
    say("glu")
    x = (RNG.standard_normal((2, 64, 1001)) * 5).astype(np.float32)
    got = run_layer(nn.GLU(dev, 32), x, dev, stream)
    assert_close(got, oracle.glu(x, axis=-2), ATOL, RTOL, "glu")


# ----------------------------------------------------------------------------- Linear
@pytest.mark.parametrize("shape,nin,nout,act", [
    ((2048, 512), 512, 2048, "none"), ((5, 7, 384), 384, 1536, "gelu"), ((300, 37), 37, 50, "relu"),
    ((130, 64), 64, 96, "sigmoid"), ((64,), 64, 33, "tanh")])
def test_linear_parity(dev, stream, shape, nin, nout, act):
    say(f"linear {shape} {nin}->{nout} {act}")
    x = RNG.standard_normal(shape).astype(np.float32)
    w = (RNG.standard_normal((nout, nin)) * 0.05).astype(np.float32)
    b = (RNG.standard_normal(nout) * 0.1).astype(np.float32)
    layer = nn.Linear(dev, nin, nout, activation=act)
    layer.load_weights(w, b)
    got = run_layer(layer, x, dev, stream)
    assert_close(got, oracle.linear(x, w, b, act=act), ATOL, RTOL, "linear")


def test_linear_closed_forms(dev, stream):
    """IntegrationTests.swift:259-324."""
    say("linear closed forms")
    l = nn.Linear(dev, 3, 2)
    l.load_weights([1, 2, 3, 4, 5, 6], [0.1, 0.2])
    np.testing.assert_allclose(run_layer(l, np.array([1.0, 2, 3]), dev, stream), [14.1, 32.2],
                               atol=1e-4)
    l2 = nn.Linear(dev, 3, 2, use_bias=False)
    l2.load_weights([1, 0, 0, 0, 1, 0])
    np.testing.assert_allclose(run_layer(l2, np.array([[1.0, 2, 3], [4, 5, 6]]), dev, stream),
                               [[1, 2], [4, 5]], atol=1e-4)


# ----------------------------------------------------------------------------- bf16 variant
# bf16-input / fp32-accumulate: operands rounded to bf16 (RNE), fp32 accumulation.
# Stated tolerances: against the oracle fed the same bf16-rounded operands, fp32 accumulation
# only -> |gpu - ref| <= 1e-4 + 1e-3 |ref|; against the fp32 oracle (the north-star bar for
# bf16 paths) -> max |gpu - ref| <= 2e-2 * max |ref|.
BF16_RTOL = 2e-2


# Per element, against the fp32 oracle: rounding x and w to bf16 (unit roundoff 2^-8) moves each
# product by at most (2^-7 + 2^-16) |x| |w|, so |gpu - ref|_ij <= 2^-7 (1.01) (|x| |w|^T)_ij plus the
# fp32 accumulation (covered by the 1e-5 term): a per-element bound on every output.
def assert_bf16_elementwise(got, x, w, ref, what):
    bound = 2.0 ** -7 * 1.01 * oracle.linear(np.abs(x), np.abs(w)) + 1e-5
    err = np.abs(np.asarray(got, np.float64) - ref)
    assert np.all(err <= bound), f"{what}: max err / bound {float((err / bound).max()):.3f}"


@pytest.mark.parametrize("shape,nin,nout,act,in_dtype", [
    ((2048, 512), 512, 2048, "none", "f32"),     # config 2 shape, fp32 input rounded on device
    ((2048, 512), 512, 2048, "none", "bf16"),    # config 2 with a bf16 input tensor
    ((300, 384), 384, 1152, "gelu", "f32"),      # ragged rows, activation epilogue
    ((7, 33, 128), 128, 96, "relu", "bf16"),     # batch dims, N not a tile multiple
    ((300, 96), 96, 64, "none", "f32"),          # K % 64 != 0: the register-staged kernel
    ((50, 96), 96, 64, "none", "bf16"),          # K % 64 != 0 with a bf16 input (widened)
])
def test_linear_bf16_parity(dev, stream, shape, nin, nout, act, in_dtype):
    from tests.conftest import assert_rel_norm
    say(f"linear bf16 {shape} {nin}->{nout} {act} input {in_dtype}")
    x = RNG.standard_normal(shape).astype(np.float32)
    w = (RNG.standard_normal((nout, nin)) * 0.02).astype(np.float32)
    b = (RNG.standard_normal(nout) * 0.1).astype(np.float32)
    layer = nn.Linear(dev, nin, nout, activation=act, precision="bf16")
    layer.load_weights(w, b)
    xt = nn.Tensor.from_numpy(dev, x, dtype=in_dtype)
    out = layer(xt, stream)
    stream.sync(60000)
    got = out.to_numpy()
    xr, wr = oracle.round_bf16(x), oracle.round_bf16(w)
    ref_rounded = oracle.linear(xr, wr, b, act=act)
    assert_close(got, ref_rounded, ATOL, RTOL, "linear bf16 vs rounded-operand oracle")
    ref = oracle.linear(x, w, b, act=act)
    assert_rel_norm(got, ref, BF16_RTOL, "linear bf16 vs fp32 oracle")
    if act == "none":
        assert_bf16_elementwise(got - b, x, w, ref - b, "linear bf16 per element")
    # and it is not silently fp32
    assert np.abs(got - ref).max() > 1e-6


def test_linear_bf16_input_tensor_f32_precision(dev, stream):
    """A bf16 input tensor into an fp32 Linear is widened exactly: the result is the fp32 GEMM of
    the rounded input."""
    say("linear f32 with a bf16 input tensor")
    x = RNG.standard_normal((64, 96)).astype(np.float32)
    w = (RNG.standard_normal((32, 96)) * 0.05).astype(np.float32)
    layer = nn.Linear(dev, 96, 32, use_bias=False)
    layer.load_weights(w)
    out = layer(nn.Tensor.from_numpy(dev, x, dtype="bf16"), stream)
    stream.sync(60000)
    assert_close(out.to_numpy(), oracle.linear(oracle.round_bf16(x), w), ATOL, RTOL,
                 "bf16 input, fp32 GEMM")
    with pytest.raises(nn.MNNError):  # other layers take f32 inputs only
        nn.LayerNorm(dev, 96)(nn.Tensor.from_numpy(dev, x, dtype="bf16"), stream)


def test_encoder_block_bf16_parity(dev, stream):
    from tests.conftest import assert_rel_norm
    say("encoder block bf16 48->96")
    x = RNG.uniform(-1, 1, (1, 48, 3001)).astype(np.float32)
    w = (RNG.standard_normal((96, 48, 8)) * np.sqrt(2 / 384)).astype(np.float32)
    b = (RNG.standard_normal(96) * 0.1).astype(np.float32)
    gm, bt = np.ones(96, np.float32), np.zeros(96, np.float32)
    rw = (RNG.standard_normal((192, 96, 1)) * np.sqrt(2 / 96)).astype(np.float32)
    rb = np.zeros(192, np.float32)
    blk = nn.UNetEncoderBlock(dev, 48, 96, 8, 4, 1, rewrite=True, precision="bf16")
    blk.load_weights(w, b, gm, bt, rw, rb)
    got = run_layer(blk, x, dev, stream)
    ref = oracle.encoder_block(x, w, b, gm, bt, 1, rewrite_w=rw, rewrite_b=rb)
    assert_rel_norm(got, ref, BF16_RTOL, "encoder block bf16")


def test_transformer_layer_bf16_parity(dev, stream):
    from tests.conftest import assert_rel_norm
    say("transformer layer bf16 (config 3 shape, seq 257)")
    cfg = workloads.config3(stress=True, seq=257)
    t = nn.TransformerLayer(dev, cfg["embed"], cfg["heads"], cfg["ffn"], precision="bf16")
    t.load_state(cfg["params"])
    got = run_layer(t, cfg["x"], dev, stream)
    ref = oracle.transformer_layer(cfg["x"], cfg["params"], cfg["heads"])
    assert_rel_norm(got, ref, BF16_RTOL, "transformer layer bf16")


def test_mha_bf16_projections_fp32_core(dev, stream):
    """MultiHeadAttention with precision bf16: the Q/K/V and output projections take bf16
    operands with fp32 accumulation and the attention core stays fp32 (the documented contract).
    The oracle rounds exactly the projection operands (x, in_proj, the attention output, out_proj)
    and keeps scores, softmax and P.V exact; a bf16 core (Q, K, P or V rounded) would move the
    outputs by ~6e-3 of their scale with these peaked scores (measured on the CPU), six times the
    1e-3 bound."""
    from tests.conftest import assert_rel_norm
    say("mha bf16: bf16 projections, fp32 core")
    E, H, B, S = 384, 8, 2, 300
    w_in = (RNG.standard_normal((3 * E, E)) * 0.1).astype(np.float32)
    b_in = (RNG.standard_normal(3 * E) * 0.05).astype(np.float32)
    w_out = (RNG.standard_normal((E, E)) * 0.05).astype(np.float32)
    b_out = (RNG.standard_normal(E) * 0.05).astype(np.float32)
    x = RNG.standard_normal((B, S, E)).astype(np.float32)
    layer = nn.MultiHeadAttention(dev, E, H, precision="bf16")
    layer.load_weights(w_in, b_in, w_out, b_out)
    got = run_layer(layer, x, dev, stream)
    r = oracle.round_bf16
    o = oracle.mha(r(x), None, r(w_in), b_in, np.eye(E), None, H)  # attention output, exact core
    ref = oracle.linear(r(o), r(w_out), b_out)
    assert_rel_norm(got, ref, 1e-3, "mha bf16 vs rounded-projection oracle")
    assert_rel_norm(got, oracle.mha(x, None, w_in, b_in, w_out, b_out, H), BF16_RTOL,
                    "mha bf16 vs fp32 oracle")
    assert np.abs(got - oracle.mha(x, None, w_in, b_in, w_out, b_out, H)).max() > 1e-5


# ----------------------------------------------------------------------------- attention
MHA_CASES = [
    # B, E, H, Sq, Sk, cross
    (1, 512, 8, 300, 300, False),     # hd 64, ragged 64-blocks
    (2, 384, 8, 200, 200, False),     # hd 48
    (1, 384, 8, 130, 257, True),      # cross, Sq != Sk
    (2, 384, 8, 700, 90, True),       # cross, short keys
    (1, 64, 4, 33, 33, False),        # hd 16 (generic kernel)
    (1, 512, 8, 1, 1, False),         # single token
    # key splits (few query workgroups, long keys): ranges merged by the combine step
    (1, 512, 8, 64, 1000, True),      # 4 ranges, ragged last block
    (2, 384, 8, 100, 777, True),      # 3 ranges, hd 48
    (1, 384, 8, 1, 2000, True),       # one query, 4 ranges
]


@pytest.mark.parametrize("case", MHA_CASES, ids=[str(c) for c in MHA_CASES])
def test_mha_parity(dev, stream, case):
    B, E, H, Sq, Sk, cross = case
    say(f"mha {case}")
    w_in = (RNG.standard_normal((3 * E, E)) * 0.05).astype(np.float32)
    b_in = (RNG.standard_normal(3 * E) * 0.05).astype(np.float32)
    w_out = (RNG.standard_normal((E, E)) * 0.05).astype(np.float32)
    b_out = (RNG.standard_normal(E) * 0.05).astype(np.float32)
    q = RNG.standard_normal((B, Sq, E)).astype(np.float32)
    kv = RNG.standard_normal((B, Sk, E)).astype(np.float32)
    layer = nn.MultiHeadAttention(dev, E, H)
    layer.load_weights(w_in, b_in, w_out, b_out)
    qt = nn.Tensor.from_numpy(dev, q)
    out = nn.Tensor(dev, q.shape)
    if cross:
        layer.forward_cross(qt, nn.Tensor.from_numpy(dev, kv), out, stream)
    else:
        layer.forward(qt, out, stream)
    stream.sync(60000)
    ref = oracle.mha(q, kv if cross else None, w_in, b_in, w_out, b_out, H)
    assert_close(out.to_numpy(), ref, ATOL, RTOL, "mha")


def test_feedforward_parity(dev, stream):
    say("feedforward")
    E, Hd = 384, 1536
    x = RNG.standard_normal((3, 257, E)).astype(np.float32)
    w1 = (RNG.standard_normal((Hd, E)) * 0.05).astype(np.float32)
    b1 = (RNG.standard_normal(Hd) * 0.05).astype(np.float32)
    w2 = (RNG.standard_normal((E, Hd)) * 0.05).astype(np.float32)
    b2 = (RNG.standard_normal(E) * 0.05).astype(np.float32)
    f = nn.FeedForward(dev, E, Hd)
    f.load_weights(w1, b1, w2, b2)
    got = run_layer(f, x, dev, stream)
    assert_close(got, oracle.feed_forward(x, w1, b1, w2, b2), ATOL, RTOL, "ffn")


# ----------------------------------------------------------------------------- blocks
@pytest.mark.parametrize("name", ["time_encoder_level0", "time_encoder_level1"])
def test_encoder_block_reference_fixture(dev, stream, golden_dir, name):
    """The reference's own fixtures (HTDemucsValidationTests.swift:37-117): abs 1e-4 or rel 1e-3."""
    say(f"encoder fixture {name}")
    d = np.load(golden_dir / f"{name}.npz")
    cin, cout, k, s, g = (int(v) for v in d["config"])
    blk = nn.UNetEncoderBlock(dev, cin, cout, k, s, g)
    blk.load_weights(d["conv_weight"], d["conv_bias"], d["norm_weight"], d["norm_bias"])
    got = run_layer(blk, d["input"], dev, stream)
    ref = d["output"].astype(np.float64)
    err = np.abs(got - ref)
    assert np.all((err <= 1e-4) | (err <= 1e-3 * np.abs(ref))), f"max abs {err.max():.3e}"


@pytest.mark.parametrize("cin,cout,L,B", [(2, 48, 5000, 1), (48, 96, 3001, 2), (192, 384, 700, 1),
                                          (8, 24, 400, 1),
                                          # fused small-input blocks: batch, ragged tile, Cin 1 / 3 / 4
                                          (2, 48, 5003, 2), (4, 32, 777, 1), (1, 16, 64, 3),
                                          (3, 48, 1031, 1),
                                          # fused first-level pass: Cin 1..4, C 48, ragged
                                          # 32-column tasks, tiny inputs, batch 3
                                          (1, 48, 777, 1), (4, 48, 2049, 2), (2, 48, 9, 3),
                                          (2, 48, 131, 1)])
def test_encoder_block_rewrite_parity(dev, stream, cin, cout, L, B):
    say(f"encoder block rewrite {cin}->{cout} L={L} B={B}")
    x = RNG.uniform(-1, 1, (B, cin, L)).astype(np.float32)
    w = (RNG.standard_normal((cout, cin, 8)) * np.sqrt(2 / (cin * 8))).astype(np.float32)
    b = (RNG.standard_normal(cout) * 0.1).astype(np.float32)
    gm = (1 + 0.1 * RNG.standard_normal(cout)).astype(np.float32)
    bt = (0.1 * RNG.standard_normal(cout)).astype(np.float32)
    rw = (RNG.standard_normal((2 * cout, cout, 1)) * np.sqrt(2 / cout)).astype(np.float32)
    rb = (RNG.standard_normal(2 * cout) * 0.1).astype(np.float32)
    blk = nn.UNetEncoderBlock(dev, cin, cout, 8, 4, 1, rewrite=True)
    blk.load_weights(w, b, gm, bt, rw, rb)
    got = run_layer(blk, x, dev, stream)
    ref = oracle.encoder_block(x, w, b, gm, bt, 1, rewrite_w=rw, rewrite_b=rb)
    assert_close(got, ref, ATOL, RTOL, "encoder block")


def test_transformer_layer_parity(dev, stream):
    say("transformer layer (config 3 shape, seq 333, stress params)")
    cfg = workloads.config3(stress=True, seq=333)
    t = nn.TransformerLayer(dev, cfg["embed"], cfg["heads"], cfg["ffn"])
    t.load_state(cfg["params"])
    got = run_layer(t, cfg["x"], dev, stream)
    assert_close(got, oracle.transformer_layer(cfg["x"], cfg["params"], cfg["heads"]), ATOL, RTOL,
                 "transformer layer")


def test_cross_transformer_parity_strong_layerscale(dev, stream):
    say("cross transformer small, LayerScale 0.5")
    cfg = workloads.config5(stress=True, batch=2, time_len=150, freq_len=301, layers=4)
    p = dict(cfg["params"])
    for k in p:
        if "gamma_" in k:
            p[k] = np.full_like(p[k], 0.5)
    ct = nn.CrossTransformerEncoder(dev, cfg["embed"], cfg["heads"], cfg["ffn"], 4, 1e-4)
    ct.load_state(p)
    tt, ft = nn.Tensor.from_numpy(dev, cfg["time"]), nn.Tensor.from_numpy(dev, cfg["freq"])
    to, fo = nn.Tensor(dev, tt.shape), nn.Tensor(dev, ft.shape)
    ct.forward_cross(tt, ft, to, fo, stream)
    stream.sync(60000)
    rt, rf = oracle.cross_transformer(cfg["time"], cfg["freq"], p, 4, cfg["heads"])
    assert_close(to.to_numpy(), rt, ATOL, RTOL, "time branch")
    assert_close(fo.to_numpy(), rf, ATOL, RTOL, "freq branch")


# The HTDemucs-structured cross transformer folds every LayerNorm into the GEMM that consumes it
# when the width is a multiple of 64 (no standalone LayerNorm launch; row statistics from the
# residual GEMMs' epilogues): LayerScale 1 so each update enters at full strength, inputs offset
# by 3 so the rows' means are large next to their spread (the folded form subtracts
# mean * sum_k W[n][k] gamma[k] from the GEMM of the raw rows), and a reload of one LayerNorm and
# one projection between forwards (the folded weights must follow). Width 96 runs the standalone
# LayerNorm kernels instead.
@pytest.mark.parametrize("E,H,ffn,offset,folded", [(384, 8, 1536, 3.0, True),
                                                   (96, 2, 192, 0.0, False)])
def test_cross_transformer_folded_layernorm(dev, stream, E, H, ffn, offset, folded):
    say(f"cross transformer E {E}: LayerNorms {'folded' if folded else 'standalone'}")
    c = workloads.config5(stress=True, batch=2, time_len=130, freq_len=257, layers=3, embed=E,
                          heads=H, ffn=ffn)
    p = {k: (np.ones_like(v) if "gamma_" in k else v) for k, v in c["params"].items()}
    t = (c["time"] + offset).astype(np.float32)
    f = (c["freq"] + offset).astype(np.float32)
    ct = nn.CrossTransformerEncoder(dev, E, H, ffn, 3, 1e-4)
    ct.load_state(p)
    tt, ft = nn.Tensor.from_numpy(dev, t), nn.Tensor.from_numpy(dev, f)
    to, fo = nn.Tensor(dev, tt.shape), nn.Tensor(dev, ft.shape)

    def run():
        ct.forward_cross(tt, ft, to, fo, stream)
        stream.sync(60000)

    names = _launch_names(dev, run)
    assert ("layernorm_f32" in names) != folded, sorted(set(names))
    if folded:
        assert names.count("ln_row_parts_f32") == 2
        assert names.count("ln_fold_f32") == 14  # per branch: 2 per self layer, 3 per cross layer
    rt, rf = oracle.cross_transformer(t, f, p, 3, H)
    assert_close(to.to_numpy(), rt, ATOL, RTOL, "time branch")
    assert_close(fo.to_numpy(), rf, ATOL, RTOL, "freq branch")
    r = np.random.Generator(np.random.PCG64(77))
    for k in ("layers.1.time.norm2.weight", "layers.1.freq.attn.in_proj_weight"):
        p[k] = (p[k] * (1 + 0.3 * r.standard_normal(p[k].shape))).astype(np.float32)
        ct.load_state({k: p[k]})
    names = _launch_names(dev, run)
    if folded:
        # time norm2 of layer 1 feeds the time KV projection; freq in_proj feeds its Q and KV
        assert names.count("ln_fold_f32") == 3
    rt, rf = oracle.cross_transformer(t, f, p, 3, H)
    assert_close(to.to_numpy(), rt, ATOL, RTOL, "time branch after reload")
    assert_close(fo.to_numpy(), rf, ATOL, RTOL, "freq branch after reload")


def test_transformer_layer_folded_layernorm(dev, stream):
    """The single transformer layer (config-3 widths, fp32) folds both LayerNorms into the GEMMs
    after them: one statistics pass over the input and no LayerNorm launch; inputs offset by 2."""
    say("transformer layer: LayerNorms folded, seq 200, offset inputs")
    cfg = workloads.config3(stress=True, seq=200)
    x = (cfg["x"] + 2.0).astype(np.float32)
    t = nn.TransformerLayer(dev, cfg["embed"], cfg["heads"], cfg["ffn"])
    t.load_state(cfg["params"])
    got = {}
    names = _launch_names(dev, lambda: got.setdefault("y", run_layer(t, x, dev, stream)))
    assert "layernorm_f32" not in names and names.count("ln_row_parts_f32") == 1, names
    assert_close(got["y"], oracle.transformer_layer(x, cfg["params"], cfg["heads"]), ATOL, RTOL,
                 "transformer layer, folded LayerNorms")


@pytest.mark.parametrize("B,St,Sf", [(1, 1, 5), (3, 2, 1)])
def test_cross_transformer_folded_layernorm_tiny(dev, stream, B, St, Sf):
    """Folded LayerNorms with fewer rows than one GEMM tile (row statistics and row coefficients
    of rows past the end are computed on clamped rows and never stored)."""
    say(f"cross transformer folded LayerNorms, tiny: B {B} time {St} freq {Sf}")
    c = workloads.config5(stress=True, batch=B, time_len=St, freq_len=Sf, layers=2)
    p = {k: (np.ones_like(v) if "gamma_" in k else v) for k, v in c["params"].items()}
    ct = nn.CrossTransformerEncoder(dev, c["embed"], c["heads"], c["ffn"], 2, 1e-4)
    ct.load_state(p)
    tt, ft = nn.Tensor.from_numpy(dev, c["time"]), nn.Tensor.from_numpy(dev, c["freq"])
    to, fo = nn.Tensor(dev, tt.shape), nn.Tensor(dev, ft.shape)
    ct.forward_cross(tt, ft, to, fo, stream)
    stream.sync(60000)
    rt, rf = oracle.cross_transformer(c["time"], c["freq"], p, 2, c["heads"])
    assert_close(to.to_numpy(), rt, ATOL, RTOL, "time branch")
    assert_close(fo.to_numpy(), rf, ATOL, RTOL, "freq branch")


@pytest.mark.parametrize("B,St,Sf,E,H,ffn,layers", [
    (2, 150, 260, 96, 2, 192, 2),    # head dim 48: the fused attention kernel
    (1, 97, 64, 64, 4, 128, 3),      # head dim 16: the generic attention kernel
    (1, 336, 672, 384, 8, 1536, 1),  # the config-5 widths
])
def test_cross_transformer_encoder_metalnn_parity(dev, stream, B, St, Sf, E, H, ffn, layers):
    """The reference-structured CrossTransformerEncoder (every layer self + cross + FFN per branch,
    one residual per sub-block, Transformer.swift:441-498) with weights loaded
    by the reference's names, against the oracle; every sub-block's update is of the order of its
    input, so a dropped or misordered term shows."""
    say(f"reference-structured cross transformer B={B} St={St} Sf={Sf} E={E} H={H} L={layers}")
    cfg = workloads.cross_encoder_metalnn(B, St, Sf, E, H, ffn, layers)
    ct = nn.MetalNNCrossTransformerEncoder(dev, E, H, ffn, layers)
    ct.load_state(cfg["params"])
    t = cfg["time"] if B > 1 else cfg["time"][0]  # [S, E] for batch 1, as the reference takes it
    f = cfg["freq"] if B > 1 else cfg["freq"][0]
    tt, ft = nn.Tensor.from_numpy(dev, t), nn.Tensor.from_numpy(dev, f)
    to, fo = nn.Tensor(dev, tt.shape), nn.Tensor(dev, ft.shape)
    ct.forward_cross(tt, ft, to, fo, stream)
    stream.sync(60000)
    rt, rf = oracle.cross_transformer_metalnn(t, f, cfg["params"], layers, H)
    assert_close(to.to_numpy(), rt, ATOL, RTOL, "time branch")
    assert_close(fo.to_numpy(), rf, ATOL, RTOL, "freq branch")


def test_cross_transformer_encoder_metalnn_errors(dev, stream):
    ct = nn.MetalNNCrossTransformerEncoder(dev, 32, 4, 64, 2)
    with pytest.raises(nn.MNNError):
        ct.load_weights_named("layers.0.norm_time_selff.weight", np.ones(32, np.float32))
    with pytest.raises(nn.MNNError):
        ct.load_weights_named("layers.2.norm_time_self.weight", np.ones(32, np.float32))
    with pytest.raises(nn.MNNError):
        nn.MetalNNCrossTransformerEncoder(dev, 30, 4, 64, 2)  # embed not divisible by heads


# ----------------------------------------------------------------------------- Sequential / errors
def test_sequential_pingpong_and_forward(dev, stream):
    """ModelTests.swift:114-162: 6 same-shape layers use <= 2 buffers; 3 shapes use 3."""
    say("sequential")
    seq = nn.Sequential(dev)
    layers = []
    for i in range(6):
        l = nn.Linear(dev, 16, 16, activation="relu" if i % 2 else "none")
        l.load_weights(RNG.standard_normal((16, 16)).astype(np.float32) * 0.3,
                       RNG.standard_normal(16).astype(np.float32) * 0.1)
        layers.append(l)
        seq.add(l)
    seq.build()
    x = RNG.standard_normal((16,)).astype(np.float32)
    out = seq.forward(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(10000)
    assert seq.buffer_stats[0] <= 2 and seq.buffer_stats[1] == 6
    assert out.to_numpy().shape == (16,)

    seq3 = nn.Sequential(dev)
    for a, b in ((8, 16), (16, 32), (32, 4)):
        seq3.add(nn.Linear(dev, a, b))
    seq3.build()
    assert seq3.buffer_stats == (3, 3)


def test_sequential_matches_oracle_chain(dev, stream):
    say("sequential numeric chain")
    ws = [(RNG.standard_normal((24, 24)) * 0.2).astype(np.float32) for _ in range(4)]
    bs = [(RNG.standard_normal(24) * 0.1).astype(np.float32) for _ in range(4)]
    seq = nn.Sequential(dev)
    keep = []
    for w, b in zip(ws, bs):
        l = nn.Linear(dev, 24, 24, activation="gelu")
        l.load_weights(w, b)
        keep.append(l)
        seq.add(l)
    seq.build()
    x = RNG.standard_normal((5, 24)).astype(np.float32)
    out = seq.forward(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(10000)
    ref = x.astype(np.float64)
    for w, b in zip(ws, bs):
        ref = oracle.linear(ref, w, b, act="gelu")
    assert_close(out.to_numpy().reshape(5, 24), ref, ATOL, RTOL, "sequential chain")


def test_sequential_errors(dev, stream):
    say("sequential errors")
    seq = nn.Sequential(dev)
    with pytest.raises(nn.MNNError) as e:
        seq.forward(nn.Tensor(dev, [4]), stream)
    assert e.value.name == "MNN_ERR_EMPTY_MODEL"
    seq.add(nn.Linear(dev, 4, 8))
    with pytest.raises(nn.MNNError) as e:
        seq.add(nn.Linear(dev, 5, 2))
    assert e.value.name == "MNN_ERR_SHAPE_MISMATCH"
    with pytest.raises(nn.MNNError) as e:
        seq.forward(nn.Tensor(dev, [4]), stream)
    # not built: invalidConfiguration("Model not built. Call build() first."), Model.swift:228-229
    assert e.value.name == "MNN_ERR_INVALID_CONFIGURATION" and "not built" in str(e.value)
    seq.build()
    with pytest.raises(nn.MNNError) as e:
        seq.forward(nn.Tensor(dev, [5]), stream)
    assert e.value.name == "MNN_ERR_INPUT_SHAPE_MISMATCH"


def test_weight_validation_errors(dev):
    say("weight validation")
    l = nn.Linear(dev, 4, 2)
    w = np.ones(8, np.float32)
    w[3] = np.nan
    with pytest.raises(nn.MNNError) as e:
        l.load_weights(w)
    assert e.value.name == "MNN_ERR_INVALID_CONFIGURATION"
    w[3] = np.inf
    with pytest.raises(nn.MNNError) as e:
        l.load_weights(w)
    assert e.value.name == "MNN_ERR_INVALID_CONFIGURATION"
    with pytest.raises(nn.MNNError) as e:
        l.load_weights(np.ones(7, np.float32))
    assert e.value.name == "MNN_ERR_BUFFER_SIZE_MISMATCH"
    with pytest.raises(nn.MNNError) as e:
        nn.MultiHeadAttention(dev, 10, 3)
    assert e.value.name == "MNN_ERR_INVALID_CONFIGURATION"


def test_shape_errors(dev, stream):
    say("shape errors")
    c = nn.DynamicConv1D(dev, 2, 4, 8, 4, padding_mode="reflect", padding=3)
    with pytest.raises(nn.MNNError) as e:
        c(nn.Tensor(dev, [3, 100]), stream)
    assert e.value.name == "MNN_ERR_SHAPE_MISMATCH"
    with pytest.raises(nn.MNNError) as e:
        c.forward(nn.Tensor(dev, [2, 100]), nn.Tensor(dev, [4, 10]), stream)
    assert e.value.name == "MNN_ERR_BUFFER_SIZE_MISMATCH"


def test_device_lost_and_stream_sync(dev):
    say("device lost")
    d2 = nn.AudioDevice(0)
    s2 = nn.Stream(d2)
    d2.check_available(2000)
    t = nn.Tensor(d2, [4])
    s2.sync(2000)
    d2.mark_lost()
    with pytest.raises(nn.MNNError) as e:
        t.copy_from(np.ones(4, np.float32))
    assert e.value.name == "MNN_ERR_DEVICE_LOST"
    with pytest.raises(nn.MNNError) as e:
        nn.Linear(d2, 2, 2)
    assert e.value.name == "MNN_ERR_DEVICE_LOST"


# ----------------------------------------------------------------------------- decoder path
@pytest.mark.parametrize("cin,cout,k,s,p,op,d,g,L,B", [
    (96, 24, 8, 4, 3, 2, 1, 1, 513, 2),    # decoder-block form (matrix cores, 2 taps per phase)
    (768, 192, 8, 4, 3, 2, 1, 1, 1344, 1),  # deepest decoder level: K split in 3 + reduce
    (384, 96, 8, 4, 3, 2, 1, 1, 300, 2),   # K split in 2, batch 2
    (20, 2, 8, 4, 3, 2, 1, 1, 1000, 1),    # 2 output channels: register kernel
    (24, 1, 8, 4, 3, 2, 1, 1, 777, 2),     # 1 output channel, batch 2
    (40, 4, 8, 4, 3, 0, 1, 1, 300, 1),     # 4 output channels, no output padding
    (20, 8, 8, 4, 3, 2, 1, 1, 1000, 1),    # padded channels, 32-row GEMM
    (64, 16, 4, 4, 0, 0, 1, 1, 300, 2),    # one tap per phase
    (16, 8, 8, 2, 1, 1, 1, 1, 77, 1),      # four taps per phase
    (8, 6, 5, 2, 1, 1, 2, 2, 50, 2),       # groups + dilation: direct kernel
    (5, 3, 3, 2, 0, 0, 1, 1, 40, 1),       # k not a multiple of the stride: direct kernel
])
def test_conv_transpose1d_parity(dev, stream, cin, cout, k, s, p, op, d, g, L, B):
    say(f"conv transpose {cin}->{cout} k{k} s{s} p{p} op{op} d{d} g{g} L={L} B={B}")
    x = RNG.standard_normal((B, cin, L)).astype(np.float32)
    w = (RNG.standard_normal((cin, cout // g, k)) / np.sqrt(cin * k / s)).astype(np.float32)
    b = (RNG.standard_normal(cout) * 0.1).astype(np.float32)
    layer = nn.ConvTranspose1D(dev, cin, cout, k, s, p, op, d, g)
    layer.load_weights(w, b)
    got = run_layer(layer, x, dev, stream)
    ref = oracle.conv_transpose1d(x, w, b, s, p, op, d, g)
    assert got.shape == ref.shape == (B, cout, layer.output_length(L))
    assert_close(got, ref, ATOL, RTOL, "conv transpose")


@pytest.mark.parametrize("cin,cskip,cout,groups,L,B,stats_pass", [
    (48, 48, 24, 8, 513, 2, True),
    (16, 16, 2, 2, 1024, 1, True),     # few-channel kernel: statistics pass
    (96, 96, 48, 8, 1344, 1, False),   # K split: the reduce writes the partials of each group
    # one group: the scatter epilogue writes one partial per tile (batch 2), the split-K reduce
    # (deepest level shape), or a statistics pass after the few-channel kernel
    (48, 48, 24, 1, 513, 2, False),
    (384, 384, 192, 1, 1344, 1, False),
    (16, 16, 2, 1, 1024, 2, True),
    (384, 384, 192, 8, 1344, 1, False),
    (192, 192, 96, 8, 2000, 2, False),
    (40, 40, 20, 5, 700, 1, True),     # five groups, no K split: statistics pass
])
def test_decoder_block_parity(dev, stream, cin, cskip, cout, groups, L, B, stats_pass):
    say(f"decoder block {cin}+{cskip}->{cout} G={groups} L={L} B={B}")
    x = RNG.standard_normal((B, cin, L)).astype(np.float32)
    sk = RNG.standard_normal((B, cskip, L)).astype(np.float32)
    w = (RNG.standard_normal((cin + cskip, cout, 8)) / np.sqrt((cin + cskip) * 2)).astype(
        np.float32)
    b = (RNG.standard_normal(cout) * 0.1).astype(np.float32)
    gm = (1 + 0.1 * RNG.standard_normal(cout)).astype(np.float32)
    bt = (0.1 * RNG.standard_normal(cout)).astype(np.float32)
    blk = nn.UNetDecoderBlock(dev, cin, cskip, cout, 8, 4, groups)
    blk.load_weights(w, b, gm, bt)
    xt, st = nn.Tensor.from_numpy(dev, x), nn.Tensor.from_numpy(dev, sk)
    res = {}

    def fwd():
        res["out"] = blk.forward_alloc(xt, st, stream)
        stream.sync(60000)
    names = _launch_names(dev, fwd)
    out = res["out"]
    # where the transposed conv writes the GroupNorm partials, no statistics pass reads its output
    assert ("gn_stats_partial" in names) == stats_pass, names
    ref = oracle.decoder_block(x, sk, w, b, gm, bt, groups)
    assert out.shape == ref.shape == (B, cout, 4 * L)
    assert_close(out.to_numpy(), ref, ATOL, RTOL, "decoder block")


def test_decoder_block_rejects_mismatched_skip(dev, stream):
    blk = nn.UNetDecoderBlock(dev, 8, 8, 4, 8, 4, 2)
    x = nn.Tensor.from_numpy(dev, np.zeros((1, 8, 32), np.float32))
    sk = nn.Tensor.from_numpy(dev, np.zeros((1, 8, 31), np.float32))
    out = nn.Tensor(dev, (1, 4, 128))
    with pytest.raises(nn.MNNError):
        blk.forward(x, sk, out, stream)
    with pytest.raises(nn.MNNError):
        blk(x, stream)  # the block needs its skip input


def test_time_unet_parity(dev, stream):
    """Two rewrite encoder levels and the two decoder levels back to the padded length
    (HTDemucs.forwardTimeUNet composition, HTDemucs.swift:521-548)."""
    left, right, L = nn.unet_padding(3000, 2, 8, 4)
    assert (left, right, L) == oracle.unet_padding(3000, 2, 8, 4)
    say(f"time U-Net 2 levels, padded length {L}")
    ch = [2, 16, 32]
    x = RNG.uniform(-1, 1, (1, 2, L)).astype(np.float32)
    enc_p, dec_p, enc, dec = [], [], [], []
    for i in range(2):
        c0, c1 = ch[i], ch[i + 1]
        lv = {"conv.weight": (RNG.standard_normal((c1, c0, 8)) * np.sqrt(2 / (8 * c0))),
              "conv.bias": RNG.standard_normal(c1) * 0.1, "norm.weight": np.ones(c1),
              "norm.bias": np.zeros(c1),
              "rewrite.weight": RNG.standard_normal((2 * c1, c1, 1)) * np.sqrt(2 / c1),
              "rewrite.bias": RNG.standard_normal(2 * c1) * 0.1}
        lv = {k: v.astype(np.float32) for k, v in lv.items()}
        blk = nn.UNetEncoderBlock(dev, c0, c1, 8, 4, 1, rewrite=True)
        blk.load_weights(lv["conv.weight"], lv["conv.bias"], lv["norm.weight"], lv["norm.bias"],
                         lv["rewrite.weight"], lv["rewrite.bias"])
        enc_p.append(lv)
        enc.append(blk)
    for i in reversed(range(2)):
        c1, c0 = ch[i + 1], ch[i]
        g = min(8, c0)
        dv = {"conv_tr.weight": (RNG.standard_normal((2 * c1, c0, 8)) / np.sqrt(4 * c1)),
              "conv_tr.bias": RNG.standard_normal(c0) * 0.1, "norm.weight": np.ones(c0),
              "norm.bias": np.zeros(c0)}
        dv = {k: v.astype(np.float32) for k, v in dv.items()}
        blk = nn.UNetDecoderBlock(dev, c1, c1, c0, 8, 4, g)
        blk.load_weights(dv["conv_tr.weight"], dv["conv_tr.bias"], dv["norm.weight"],
                         dv["norm.bias"])
        dv["groups"] = g
        dec_p.append(dv)
        dec.append(blk)
    y = nn.Tensor.from_numpy(dev, x)
    skips = []
    for blk in enc:
        y = blk(y, stream)
        skips.append(y)
    for i, blk in enumerate(dec):
        y = blk.forward_alloc(y, skips[len(skips) - 1 - i], stream)
    stream.sync(60000)
    ref = oracle.time_unet(x, enc_p, dec_p)
    assert y.shape == ref.shape == (1, 2, L)
    assert_close(y.to_numpy(), ref, ATOL, RTOL, "time U-Net")


def test_layer_weights_from_safetensors(dev, stream, tmp_path):
    """A rewrite encoder block loaded from a SafeTensors file (F32 and F16 entries) matches the
    oracle on the file's values (SafeTensorsLoader.loadTensor(name:into:))."""
    from safetensors.numpy import save_file
    say("encoder block weights from safetensors")
    cin, cout, L = 2, 16, 999
    w = {"enc.0.conv.weight": (RNG.standard_normal((cout, cin, 8)) * 0.3).astype(np.float32),
         "enc.0.conv.bias": (RNG.standard_normal(cout) * 0.1).astype(np.float32),
         "enc.0.norm.weight": (1 + 0.1 * RNG.standard_normal(cout)).astype(np.float16),
         "enc.0.norm.bias": (0.1 * RNG.standard_normal(cout)).astype(np.float16),
         "enc.0.rewrite.weight": (RNG.standard_normal((2 * cout, cout, 1)) * 0.3).astype(np.float32),
         "enc.0.rewrite.bias": (RNG.standard_normal(2 * cout) * 0.1).astype(np.float32)}
    save_file(w, str(tmp_path / "enc.safetensors"))
    st = nn.SafeTensors(tmp_path / "enc.safetensors")
    blk = nn.UNetEncoderBlock(dev, cin, cout, 8, 4, 1, rewrite=True)
    for k in w:
        st.load_into(blk, k, k[len("enc.0."):])
    x = RNG.uniform(-1, 1, (1, cin, L)).astype(np.float32)
    got = run_layer(blk, x, dev, stream)
    f = {k: v.astype(np.float32) for k, v in w.items()}
    ref = oracle.encoder_block(x, f["enc.0.conv.weight"], f["enc.0.conv.bias"],
                               f["enc.0.norm.weight"], f["enc.0.norm.bias"], 1,
                               rewrite_w=f["enc.0.rewrite.weight"],
                               rewrite_b=f["enc.0.rewrite.bias"])
    assert_close(got, ref, ATOL, RTOL, "encoder block from safetensors")
    with pytest.raises(nn.MNNError):
        st.load_into(blk, "enc.0.conv.bias", "conv.weight")  # wrong element count


@pytest.mark.gpu
def test_layer_weights_from_mtla(dev, stream, tmp_path):
    """A 1x1-GLU encoder block loaded from an "MTLA" model file written by BinaryModelFile.save
    matches the oracle on the same values (BinaryModelLoader.load, Model.swift:466-622)."""
    say("encoder block weights from an MTLA file")
    cin, cout, L = 2, 16, 777
    w = {"conv.weight": (RNG.standard_normal((cout, cin, 8)) * 0.3).astype(np.float32),
         "conv.bias": (RNG.standard_normal(cout) * 0.1).astype(np.float32),
         "norm.weight": (1 + 0.1 * RNG.standard_normal(cout)).astype(np.float32),
         "norm.bias": (0.1 * RNG.standard_normal(cout)).astype(np.float32),
         "rewrite.weight": (RNG.standard_normal((2 * cout, cout, 1)) * 0.3).astype(np.float32),
         "rewrite.bias": (RNG.standard_normal(2 * cout) * 0.1).astype(np.float32)}
    nn.BinaryModelFile.save(w, tmp_path / "enc.bin")
    m = nn.BinaryModelFile(tmp_path / "enc.bin")
    blk = nn.UNetEncoderBlock(dev, cin, cout, 8, 4, 1, rewrite=True)
    for k in m.names:
        m.load_into(blk, k, k)
    x = RNG.uniform(-1, 1, (1, cin, L)).astype(np.float32)
    got = run_layer(blk, x, dev, stream)
    ref = oracle.encoder_block(x, w["conv.weight"], w["conv.bias"], w["norm.weight"],
                               w["norm.bias"], 1, rewrite_w=w["rewrite.weight"],
                               rewrite_b=w["rewrite.bias"])
    assert_close(got, ref, ATOL, RTOL, "encoder block from MTLA")
    with pytest.raises(nn.MNNError):
        m.load_into(blk, "conv.bias", "conv.weight")  # wrong element count


# ----------------------------------------------------------------------------- FusedConv1D residual
# (B, cin, cout, k, s, p, g, act, alpha, L): the direct kernels (small contractions, groups) and
# the matrix-core implicit GEMM (Cin * K >= 64); biases are negative so that many pre-activations
# are negative: a residual added before ReLU / leaky ReLU instead of after fails these.
FUSED_CASES = [
    (1, 2, 48, 8, 4, 0, 1, "relu", 0.01, 4001),          # register-window direct kernel
    (2, 6, 12, 5, 2, 2, 3, "leaky_relu", 0.25, 203),     # generic direct kernel, groups
    (2, 48, 96, 8, 4, 3, 1, "relu", 0.01, 1031),         # implicit GEMM on the matrix cores
    (1, 96, 64, 4, 1, 1, 1, "leaky_relu", 0.2, 517),     # implicit GEMM, leaky slope 0.2
    (1, 16, 32, 3, 1, 1, 1, "gelu", 0.01, 300),
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=[str(c) for c in FUSED_CASES])
def test_fused_conv1d_residual_parity(dev, stream, case):
    B, cin, cout, k, s, p, g, act, alpha, L = case
    say(f"fused conv1d residual {case}")
    x = RNG.uniform(-1, 1, (B, cin, L)).astype(np.float32)
    w = (RNG.standard_normal((cout, cin // g, k)) * np.sqrt(2 / (cin // g * k))).astype(np.float32)
    b = (RNG.standard_normal(cout) * 0.1 - 0.3).astype(np.float32)
    layer = nn.FusedConv1D(dev, cin, cout, k, s, p, groups=g, activation=act,
                           leaky_relu_alpha=alpha)
    layer.load_weights(w, b)
    lo = (L + 2 * p - k) // s + 1
    res = (RNG.standard_normal((B, cout, lo)) * 2).astype(np.float32)
    xt, rt = nn.Tensor.from_numpy(dev, x), nn.Tensor.from_numpy(dev, res)
    out = nn.Tensor(dev, (B, cout, lo))
    layer.forward_with_residual(xt, rt, out, stream)
    stream.sync(60000)
    ref = oracle.fused_conv1d(x, w, b, stride=s, padding=p, groups=g, act=act, alpha=alpha,
                              residual=res)
    pre = oracle.conv1d(x, w, b, stride=s, padding=p, groups=g)
    assert (pre < 0).mean() > 0.2  # the activation's negative side is exercised
    assert_close(out.to_numpy(), ref, ATOL, RTOL, "fused conv + residual")
    # residual = output (in place) and no residual
    out2 = nn.Tensor.from_numpy(dev, res)
    layer.forward_with_residual(xt, out2, out2, stream)
    layer.forward_with_residual(xt, None, out, stream)
    stream.sync(60000)
    assert_close(out2.to_numpy(), ref, ATOL, RTOL, "fused conv + residual in place")
    assert_close(out.to_numpy(), oracle.activation(pre, act, alpha=alpha), ATOL, RTOL,
                 "fused conv without residual")


def test_fused_conv1d_residual_errors(dev, stream):
    say("fused conv residual errors")
    layer = nn.FusedConv1D(dev, 4, 8, 3, padding=1)
    x = nn.Tensor(dev, (1, 4, 20))
    with pytest.raises(nn.MNNError) as e:
        layer.forward_with_residual(x, nn.Tensor(dev, (1, 8, 19)), nn.Tensor(dev, (1, 8, 20)),
                                    stream)
    assert e.value.name == "MNN_ERR_BUFFER_SIZE_MISMATCH"
    with pytest.raises(nn.MNNError) as e:
        gn = nn.GroupNorm(dev, 1, 4)
        nn.Conv1D.forward_with_residual(gn, x, None, nn.Tensor(dev, (1, 4, 20)), stream)
    assert e.value.name == "MNN_ERR_INVALID_ARGUMENT"
    for xi, ri in ((nn.Tensor(dev, (1, 4, 20), dtype="bf16"), None),  # 2-byte elements
                   (x, nn.Tensor(dev, (1, 8, 20), dtype="bf16"))):
        with pytest.raises(nn.MNNError) as e:
            layer.forward_with_residual(xi, ri, nn.Tensor(dev, (1, 8, 20)), stream)
        assert e.value.name == "MNN_ERR_INVALID_ARGUMENT"
    with pytest.raises(nn.MNNError):
        nn.FusedConv1D(dev, 4, 8, 3, leaky_relu_alpha=float("nan"))


def test_fused_linear_leaky_alpha(dev, stream):
    say("fused linear leaky relu alpha 0.3")
    x = RNG.standard_normal((300, 64)).astype(np.float32)
    w = (RNG.standard_normal((96, 64)) * 0.1).astype(np.float32)
    b = (RNG.standard_normal(96) * 0.1).astype(np.float32)
    layer = nn.FusedLinear(dev, 64, 96, activation="leaky_relu", leaky_relu_alpha=0.3)
    layer.load_weights(w, b)
    got = run_layer(layer, x, dev, stream)
    assert_close(got, oracle.linear(x, w, b, act="leaky_relu", alpha=0.3), ATOL, RTOL,
                 "fused linear alpha")


# ----------------------------------------------------------------------------- Sequential API
def test_sequential_layer_at(dev):
    """layer(at:) (Model.swift:354-357): the added layers in order, None out of range."""
    say("sequential layer(at:)")
    seq = nn.Sequential(dev)
    ls = [nn.Linear(dev, 8, 8) for _ in range(3)]
    for l in ls:
        seq.add(l)
    assert seq.layer_count == 3
    assert [seq.layer(i) for i in range(3)] == ls
    assert seq.layer(3) is None and seq.layer(-1) is None


def test_sequential_forward_async(dev, stream):
    """forwardAsync (Model.swift:271-346): the completion gets the same output forward() gives,
    once; failures before enqueueing reach the completion on the calling thread."""
    import threading
    say("sequential forwardAsync")
    seq = nn.Sequential(dev)
    keep = []
    for _ in range(3):
        l = nn.Linear(dev, 32, 32, activation="gelu")
        l.load_weights((RNG.standard_normal((32, 32)) * 0.2).astype(np.float32),
                       (RNG.standard_normal(32) * 0.1).astype(np.float32))
        keep.append(l)
        seq.add(l)
    seq.build()
    x = RNG.standard_normal((50, 32)).astype(np.float32)
    xt = nn.Tensor.from_numpy(dev, x)
    want = seq.forward(xt, stream).to_numpy(stream).copy()
    done = threading.Event()
    got = {}

    def completion(status, out):
        got["status"] = status
        got["value"] = out.to_numpy() if out is not None else None
        got["thread"] = threading.get_ident()
        got["calls"] = got.get("calls", 0) + 1
        done.set()

    rc = seq.forward_async(xt, completion, stream)
    assert rc == 0
    assert done.wait(30), "completion not called"
    assert got["status"] == 0 and got["calls"] == 1
    assert got["thread"] != threading.get_ident()
    np.testing.assert_array_equal(got["value"], want)
    # a completion may start the next forwardAsync (the in-flight mark is already cleared)
    done2 = threading.Event()
    chained = {}

    def second(status, out):
        chained["status"] = status
        done2.set()

    def first(status, out):
        chained["rc"] = seq.forward_async(xt, second, stream)

    assert seq.forward_async(xt, first, stream) == 0
    assert done2.wait(30) and chained["rc"] == 0 and chained["status"] == 0
    # a completion may destroy its own model: the destroy returns (it does not wait for the
    # completion that called it) and the library thread ends without touching the model
    gone = nn.Sequential(dev)
    gone.add(keep[0])
    gone.build()
    done3 = threading.Event()
    closed = {}

    def closing(status, out):
        closed["status"] = status
        gone.close()
        closed["handle"] = gone.handle
        done3.set()

    assert gone.forward_async(xt, closing, stream) == 0
    assert done3.wait(30) and closed == {"status": 0, "handle": None}
    # not built / empty: reported through the completion, synchronously, and returned
    errs = []
    empty = nn.Sequential(dev)
    rc = empty.forward_async(xt, lambda st, out: errs.append((st, out)), stream)
    assert rc == 9 and errs == [(9, None)]  # MNN_ERR_EMPTY_MODEL
    unbuilt = nn.Sequential(dev)
    unbuilt.add(nn.Linear(dev, 32, 32))
    rc = unbuilt.forward_async(xt, lambda st, out: errs.append((st, out)), stream)
    assert rc == 1 and errs[-1] == (1, None)  # invalidConfiguration, as Model.swift:293-298


@pytest.mark.parametrize("cin,cout,L,act,gelu,k,mode,pad", [
    (2, 48, 44100, "none", True, 8, "reflect", 3),   # config-1 shape: register-window, GELU fused
    (48, 96, 3001, "none", False, 8, "reflect", 3),  # matrix-core conv with GEMM statistics
    (8, 16, 777, "gelu", False, 4, "reflect", 3),    # GroupNorm's own fused activation
    (1, 16, 5003, "relu", False, 8, "explicit", 2),  # zero padding, ReLU, ragged last workgroup
    (3, 32, 2999, "leaky_relu", False, 8, "explicit", 5),  # Cin * K = 24
    (4, 64, 1025, "sigmoid", False, 8, "reflect", 3),      # Cin * K = 32
    (2, 24, 301, "tanh", False, 4, "explicit", 1),         # Cin * K = 8, three channel blocks
    (2, 48, 343980, "none", True, 8, "reflect", 3),  # grid too large for one launch: two passes
])
def test_sequential_conv_groupnorm_fusion(dev, stream, cin, cout, L, act, gelu, k, mode, pad):
    """Conv1D -> GroupNorm(1) [-> activation / GELU] in a Sequential runs fused (one launch when
    the grid fits the device at once, else two); the result is the layers' composition, batch 2
    included. The bias and GroupNorm shift carry an offset so that a dropped bias or mean term
    moves the output."""
    say(f"sequential conv -> groupnorm fusion {cin}->{cout} k{k} L={L} {mode} act={act} "
        f"gelu={gelu}")
    x = RNG.uniform(-1, 1, (2, cin, L)).astype(np.float32)
    w = (RNG.standard_normal((cout, cin, k)) * np.sqrt(2 / (cin * k))).astype(np.float32)
    b = (0.5 + RNG.standard_normal(cout) * 0.3).astype(np.float32)
    gm = (1 + 0.2 * RNG.standard_normal(cout)).astype(np.float32)
    bt = (0.2 * RNG.standard_normal(cout)).astype(np.float32)
    conv = nn.DynamicConv1D(dev, cin, cout, k, 4, padding_mode=mode, padding=pad)
    conv.load_weights(w, b)
    gn = nn.GroupNorm(dev, 1, cout, activation=act)
    gn.load_parameters(gm, bt)
    seq = nn.Sequential(dev)
    seq.add(conv)
    seq.add(gn)
    layers = [conv, gn]
    if gelu:
        g = nn.GELU(dev, [cout, 0])
        seq.add_unchecked(g)
        layers.append(g)
    seq.build()
    out = seq.forward(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(60000)
    ref = oracle.group_norm(oracle.conv1d(x, w, b, stride=4, padding=pad,
                                          mode="reflect" if mode == "reflect" else "zeros"),
                            1, gm, bt)
    ref = oracle.gelu_layer(ref) if gelu else oracle.activation(ref, act)
    assert_close(out.to_numpy().reshape(ref.shape), ref, ATOL, RTOL, "fused sequential")


@pytest.mark.parametrize("C,L", [(16, 20001), (32, 4099)])
def test_sequential_fused_chain_output_aliases_its_input(dev, stream, C, L):
    """GELU -> Conv1D(C -> C, k 1) -> GroupNorm(1): the ping-pong plan gives GroupNorm (the fused
    chain's last layer) the buffer GELU wrote, i.e. the chain's own input. The result must still be
    the layers' composition (the chain then goes through the conv's own buffer)."""
    say(f"fused chain whose output aliases its input C={C} L={L}")
    x = RNG.uniform(-2, 2, (C, L)).astype(np.float32)
    w = (RNG.standard_normal((C, C, 1)) * np.sqrt(2 / C)).astype(np.float32)
    b = (0.5 + 0.3 * RNG.standard_normal(C)).astype(np.float32)
    gm = (1 + 0.2 * RNG.standard_normal(C)).astype(np.float32)
    bt = (0.2 * RNG.standard_normal(C)).astype(np.float32)
    seq = nn.Sequential(dev)
    seq.add(nn.GELU(dev, [C, L]))
    conv = nn.Conv1D(dev, C, C, 1, input_length=L)
    conv.load_weights(w, b)
    seq.add(conv)
    gn = nn.GroupNorm(dev, 1, C, activation="relu")
    gn.load_parameters(gm, bt)
    seq.add_unchecked(gn)
    seq.build()
    assert seq.buffer_stats == (2, 3)  # GroupNorm reuses GELU's buffer
    out = seq.forward(nn.Tensor.from_numpy(dev, x), stream)
    stream.sync(60000)
    ref = oracle.activation(oracle.group_norm(oracle.conv1d(oracle.gelu_layer(x), w, b), 1, gm,
                                              bt), "relu")
    assert_close(out.to_numpy().reshape(ref.shape), ref, ATOL, RTOL, "aliased fused chain")


def _launch_names(dev, fn):
    """Kernel names launched on `dev` while fn() runs, in launch order."""
    lib = _lib.lib()
    assert lib.mnn_debug_set_launch_log(dev.handle, 1) == 0
    try:
        fn()
    finally:
        lib.mnn_debug_set_launch_log(dev.handle, 0)
    need = ctypes.c_size_t()
    lib.mnn_debug_launch_log(dev.handle, None, 0, ctypes.byref(need))
    buf = ctypes.create_string_buffer(need.value)
    assert lib.mnn_debug_launch_log(dev.handle, buf, need.value, ctypes.byref(need)) == 0
    return [ln.split()[0] for ln in buf.value.decode().splitlines() if ln.strip()]


def _spin_limit(dev, polls):
    prev = ctypes.c_int()
    assert _lib.lib().mnn_debug_set_grid_spin_limit(dev.handle, polls, ctypes.byref(prev)) == 0
    return prev.value


def test_conv_groupnorm_one_launch(dev, stream):
    """The config-1 chain (Conv1D 2->48 k8 s4 -> GroupNorm(1) -> GELU) runs as one launch whose
    workgroups wait for each other's statistics. Checked: the launch count; the oracle; repeated
    calls and a shorter input in between (the arrival counters return to zero after each launch,
    and the partial count follows the grid); the bounded wait's other path, forced from the host
    with a spin limit of 0 (workgroups that arrive before the last one compute every partial
    themselves), which gives the same bits; and a grid too large for the device going to the
    two-launch form."""
    say("conv -> groupnorm one launch: config-1 chain, spin limit default and 0")
    x = RNG.uniform(-1, 1, (1, 2, 44100)).astype(np.float32)
    xs = RNG.uniform(-1, 1, (1, 2, 9000)).astype(np.float32)
    w = (RNG.standard_normal((48, 2, 8)) * 0.5).astype(np.float32)
    b = (0.3 + 0.2 * RNG.standard_normal(48)).astype(np.float32)
    gm = (1 + 0.2 * RNG.standard_normal(48)).astype(np.float32)
    bt = (0.2 * RNG.standard_normal(48)).astype(np.float32)
    conv = nn.Conv1D(dev, 2, 48, 8, 4)
    conv.load_weights(w, b)
    gn = nn.GroupNorm(dev, 1, 48)
    gn.load_parameters(gm, bt)
    seq = nn.Sequential(dev)
    seq.add(conv)
    seq.add(gn)
    seq.add_unchecked(nn.GELU(dev, [48, 0]))
    seq.build()

    def ref(xx):
        return oracle.gelu_layer(oracle.group_norm(oracle.conv1d(xx, w, b, stride=4), 1, gm, bt))

    def run(xx):
        o = seq.forward(nn.Tensor.from_numpy(dev, xx), stream)
        stream.sync(60000)
        return o.to_numpy().reshape(1, 48, -1)

    r, rs = ref(x), ref(xs)
    # the first call also zeroes the layer's arrival counters (a kernel of its own)
    names = _launch_names(dev, lambda: run(x))
    assert names == ["zero_u32", "conv_gn_oneshot_f32"], names
    names = _launch_names(dev, lambda: run(x))
    assert names == ["conv_gn_oneshot_f32"], names
    first = run(x)
    assert_close(first, r, ATOL, RTOL, "one launch")
    for _ in range(3):
        assert_close(run(xs), rs, ATOL, RTOL, "one launch, shorter input")
        assert np.array_equal(run(x), first), "repeated one-launch calls differ"
    prev = _spin_limit(dev, 0)
    try:
        assert prev > 0
        for _ in range(2):
            assert np.array_equal(run(x), first), "self-computed statistics differ"
            assert_close(run(xs), rs, ATOL, RTOL, "self-computed statistics, shorter input")
    finally:
        _spin_limit(dev, prev)
    assert np.array_equal(run(x), first)
    # batch 8 of 343 980 samples: 336 x 6 x 8 workgroups, more than the device holds at once
    xb = RNG.uniform(-1, 1, (8, 2, 343980)).astype(np.float32)
    names = _launch_names(dev, lambda: run_batch(seq, dev, stream, xb))
    assert names == ["conv_gn_stats_f32", "conv_gn_apply_f32"], names
    assert _lib.lib().mnn_debug_set_grid_spin_limit(dev.handle, -1, None) == 12  # invalid


def run_batch(seq, dev, stream, xx):
    o = seq.forward(nn.Tensor.from_numpy(dev, xx), stream)
    stream.sync(60000)
    return o


@pytest.mark.parametrize("cin,cout,L,Ls,B", [
    (2, 48, 343980, 20001, 1),  # first level (config 4): conv, GroupNorm, GELU, rewrite in one launch
    (96, 192, 21499, 5003, 1),  # split-K conv + one-launch finish (config 4's third level)
    (192, 384, 5375, 777, 2),   # fourth level's shape, batch 2
])
def test_encoder_one_launch_groupnorm(dev, stream, cin, cout, L, Ls, B):
    """The encoder block's GroupNorm(1) forms whose workgroups exchange their statistics: the first
    level in one launch (no statistics pass) and the split-K finish of the deeper levels (no
    pre-norm y in HBM, no normalisation pass). Checked: the launches; the oracle; repeated calls
    with a shorter input in between (the exchange buffer returns to zero after each launch); and
    the bounded wait's other path, forced with a spin limit of 0 (workgroups that arrive before the
    last one compute every partial themselves), which gives the same bits."""
    say(f"encoder one-launch GroupNorm {cin}->{cout} L={L} B={B}, spin limit default and 0")
    x = RNG.uniform(-1, 1, (B, cin, L)).astype(np.float32)
    xs = RNG.uniform(-1, 1, (B, cin, Ls)).astype(np.float32)
    w = (RNG.standard_normal((cout, cin, 8)) * np.sqrt(2 / (cin * 8))).astype(np.float32)
    b = (0.3 + 0.1 * RNG.standard_normal(cout)).astype(np.float32)
    gm = (1 + 0.1 * RNG.standard_normal(cout)).astype(np.float32)
    bt = (0.1 * RNG.standard_normal(cout)).astype(np.float32)
    rw = (RNG.standard_normal((2 * cout, cout, 1)) * np.sqrt(2 / cout)).astype(np.float32)
    rb = (RNG.standard_normal(2 * cout) * 0.1).astype(np.float32)
    blk = nn.UNetEncoderBlock(dev, cin, cout, 8, 4, 1, rewrite=True)
    blk.load_weights(w, b, gm, bt, rw, rb)

    def run(xx):
        return run_layer(blk, xx, dev, stream)

    names = _launch_names(dev, lambda: run(x))
    tag = f"[c{cout}]"
    if cin <= 4:
        assert names == ["zero_u32", "enc_l1_oneshot_f32" + tag], names
    else:
        assert names == ["zero_u32", "enc_conv_f32" + tag, "enc_conv_reduce_gn_f32" + tag,
                         "enc_rewrite_f32" + tag], names
    first = run(x)
    assert_close(first, oracle.encoder_block(x, w, b, gm, bt, 1, rewrite_w=rw, rewrite_b=rb),
                 ATOL, RTOL, "one-launch GroupNorm")
    rs = oracle.encoder_block(xs, w, b, gm, bt, 1, rewrite_w=rw, rewrite_b=rb)
    first_s = run(xs)
    assert_close(first_s, rs, ATOL, RTOL, "one-launch GroupNorm, shorter input")
    for _ in range(2):
        assert np.array_equal(run(x), first), "repeated one-launch calls differ"
        assert np.array_equal(run(xs), first_s), "repeated one-launch calls differ (shorter)"
    # self-computed statistics: the first level at full size too (two tasks per wave); the split-K
    # finish on the shorter input (a workgroup that computes every partial reads every K part)
    prev = _spin_limit(dev, 0)
    try:
        assert prev > 0
        assert np.array_equal(run(xs), first_s), "self-computed statistics differ"
        if cin <= 4:
            assert np.array_equal(run(x), first), "self-computed statistics differ (full size)"
    finally:
        _spin_limit(dev, prev)
    assert np.array_equal(run(x), first)
