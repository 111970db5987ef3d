"""Pins of the oracle's frequency-branch functions (conv2d, conv_transpose2d, the 2-D U-Net
blocks and padding): the reference's own fixtures (Conv2DReference/*.json and
HTDemucsReference/freq_encoder_level{0,1}.json, converted by tests/golden/make_fixtures.py) at
the reference's tolerance, PyTorch's CPU conv2d / conv_transpose2d (a library routine) over
configurations the fixtures leave open (groups, dilation, non-square strides, reflect and
"same" padding), and closed forms for the padding calculator."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from metalaudio_amd import nn
from tests.conftest import assert_close

RNG = np.random.default_rng(41)
CASES = ["1x1_pointwise", "3x3_asymmetric_input", "3x3_no_bias", "3x3_same_padding",
         "3x3_stride2_htdemucs", "basic_3x3_no_padding", "conv_transpose_basic",
         "conv_transpose_htdemucs", "identity_like"]


@pytest.fixture(scope="module")
def conv2d_ref(golden_dir):
    return np.load(golden_dir / "conv2d_reference.npz")


def case(z, name):
    cfg = z[f"{name}/config"]
    bias = z[f"{name}/bias"] if f"{name}/bias" in z.files else None
    return z[f"{name}/input"], z[f"{name}/weight"], bias, z[f"{name}/output"], cfg


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_conv2d_fixtures(conv2d_ref, name):
    x, w, b, want, cfg = case(conv2d_ref, name)
    cin, cout, kh, kw, sh, sw, ph, pw, oph, opw, dh, dw, groups, transposed = cfg
    if transposed:
        got = oracle.conv_transpose2d(x, w, b, (sh, sw), (ph, pw), (oph, opw), (dh, dw), groups)
    else:
        got = oracle.conv2d(x, w, b, (sh, sw), "explicit", (ph, pw), (dh, dw), groups)
    assert got.shape == want.shape
    assert_close(got, want, 1e-4, 1e-3, name)


@pytest.mark.parametrize("level", [0, 1])
def test_oracle_matches_freq_encoder_fixtures(golden_dir, level):
    z = np.load(golden_dir / f"freq_encoder_level{level}.npz")
    cin, cout, kh, kw, sh, sw, groups = z["config"]
    got = oracle.freq_encoder_block(z["input"], z["conv_weight"], z["conv_bias"],
                                    z["norm_weight"], z["norm_bias"], groups, (kh, kw), (sh, sw))
    assert got.shape == z["output"].shape
    assert_close(got, z["output"], 1e-4, 1e-3, f"freq encoder level {level}")


@pytest.mark.parametrize("B,cin,cout,H,W,k,s,mode,pad,d,g", [
    (2, 4, 6, 9, 7, (3, 2), (2, 1), "explicit", (1, 1), (1, 2), 2),
    (1, 3, 5, 8, 6, (3, 3), (2, 2), "reflect", (1, 1), (1, 1), 1),
    (1, 3, 4, 11, 10, (8, 1), (4, 1), "reflect", (3, 0), (1, 1), 1),
    (2, 2, 4, 7, 9, (3, 3), (1, 1), "same", (0, 0), (1, 1), 1),
    (1, 6, 6, 10, 10, (3, 3), (2, 2), "same", (0, 0), (2, 2), 3),
    (1, 2, 3, 5, 5, (2, 2), (1, 1), "valid", (0, 0), (1, 1), 1),
])
def test_oracle_conv2d_matches_torch(B, cin, cout, H, W, k, s, mode, pad, d, g):
    x = RNG.standard_normal((B, cin, H, W))
    w = RNG.standard_normal((cout, cin // g, *k))
    b = RNG.standard_normal(cout)
    got = oracle.conv2d(x, w, b, s, mode, pad, d, g)
    ph, pw = oracle.layers.conv2d_padding(H, W, k, s, mode, pad, d)
    xt = torch.tensor(x)
    if mode == "reflect":
        xt = F.pad(xt, (pw, pw, ph, ph), mode="reflect")
        ph = pw = 0
    want = F.conv2d(xt, torch.tensor(w), torch.tensor(b), s, (ph, pw), d, g).numpy()
    assert got.shape == want.shape == (B, cout, *oracle.conv2d_output_size(H, W, k, s, mode, pad, d))
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_oracle_same_padding_quirk():
    """"same" pads total/2 on both sides (computePadding :226-236): with an even kernel the output
    is one short of ceil(n/s), as the reference computes it."""
    assert oracle.conv2d_output_size(8, 8, (2, 2), (1, 1), "same") == (7, 7)
    assert oracle.conv2d_output_size(8, 8, (3, 3), (1, 1), "same") == (8, 8)
    assert oracle.conv2d_output_size(9, 9, (3, 3), (2, 2), "same") == (5, 5)


def test_reflect_index_clamps_like_the_reference():
    n = 4
    assert list(oracle.reflect_index(np.arange(-3, 8), n)) == [3, 2, 1, 0, 1, 2, 3, 2, 1, 0, 0]


@pytest.mark.parametrize("B,cin,cout,H,W,k,s,p,op,d,g", [
    (2, 6, 6, 5, 4, (3, 4), (2, 3), (1, 2), (1, 2), (1, 1), 2),
    (1, 4, 3, 3, 5, (3, 3), (2, 2), (1, 1), (1, 1), (1, 1), 1),
    (1, 4, 2, 4, 3, (8, 1), (4, 1), (2, 0), (0, 0), (1, 1), 1),
    (2, 2, 4, 6, 6, (3, 3), (1, 2), (0, 1), (0, 1), (2, 1), 2),
])
def test_oracle_conv_transpose2d_matches_torch(B, cin, cout, H, W, k, s, p, op, d, g):
    x = RNG.standard_normal((B, cin, H, W))
    w = RNG.standard_normal((cin, cout // g, *k))
    b = RNG.standard_normal(cout)
    got = oracle.conv_transpose2d(x, w, b, s, p, op, d, g)
    want = F.conv_transpose2d(torch.tensor(x), torch.tensor(w), torch.tensor(b), s, p, op, g,
                              d).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_oracle_freq_decoder_block_matches_torch():
    x = RNG.standard_normal((2, 6, 4, 5))
    sk = RNG.standard_normal((2, 6, 4, 5))
    w = RNG.standard_normal((12, 8, 3, 3)) * 0.2
    b, gm, bt = RNG.standard_normal(8) * 0.1, 1 + 0.1 * RNG.standard_normal(8), RNG.standard_normal(8) * 0.1
    got = oracle.freq_decoder_block(x, sk, w, b, gm, bt, 4)
    t = F.conv_transpose2d(torch.cat([torch.tensor(x), torch.tensor(sk)], 1), torch.tensor(w),
                           torch.tensor(b), 2, 1, 1)
    t = F.group_norm(t, 4, torch.tensor(gm), torch.tensor(bt), 1e-5)
    want = F.gelu(t, approximate="tanh").numpy()
    assert got.shape == (2, 8, 8, 10)
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("H,W,levels,stride", [(2049, 100, 4, 2), (64, 32, 2, 2), (5, 7, 1, 3),
                                               (2048, 336, 4, 4), (1, 1, 0, 2)])
def test_padding_2d_closed_form(H, W, levels, stride):
    t, bt, l, r, oh, ow = oracle.unet_padding_2d(H, W, levels, stride)
    div = stride ** levels
    assert oh % div == 0 and ow % div == 0 and 0 <= oh - H < div and 0 <= ow - W < div
    assert t + bt == oh - H and l + r == ow - W and t == (oh - H) // 2 and l == (ow - W) // 2
    assert nn.unet_padding_2d(H, W, levels, stride) == (t, bt, l, r, oh, ow)
    bh, bw = nn.unet_bottleneck_2d(oh, ow, levels, stride)
    assert (bh, bw) == (oh // div, ow // div)
