"""Pins of the separation oracle: the segment driver's crossfade by invariants and closed forms
(an identity segment function reproduces the input exactly, since the blend weights sum to one;
constant segments give the linear ramp (i + 1) / (F + 1)), and the time-domain model by
composition of the already pinned layer oracles plus closed forms of the de-interleave / crop
(an all-zero network gives each head's bias; the padding is UNetPaddingCalculator's)."""
import numpy as np
import pytest

from oracle import layers as ol
from oracle import separate as osep

RNG = np.random.default_rng(71)


@pytest.mark.parametrize("n,seg,ovl", [(1000, 300, 50), (1000, 300, 0), (997, 250, 249),
                                       (100, 100, 10), (100, 0, 0), (1000, 999, 998)])
def test_driver_identity_invariant(n, seg, ovl):
    x = RNG.standard_normal(n * 2)
    out = osep.separate_long(x, 2, seg, ovl, lambda s: np.stack([s, -s]))
    np.testing.assert_allclose(out[0], x, atol=1e-12)
    np.testing.assert_allclose(out[1], -x, atol=1e-12)


def test_driver_ramp_closed_form():
    calls = []

    def fn(s):
        calls.append(len(s) // 2)
        return np.full((1, len(s)), float(len(calls)))
    out = osep.separate_long(np.zeros(2 * 10), 2, 6, 3, fn).reshape(10, 2)[:, 0]
    # segments [0,6) -> 1, [3,9) -> 2 over frames 3..5 with weights 1/4, 2/4, 3/4, [6,10) -> 3
    # over frames 6..8
    assert calls == [6, 6, 4]
    want = [1, 1, 1, 1.25, 1.5, 1.75, 2 + 0.25, 2 + 0.5, 2 + 0.75, 3]
    np.testing.assert_allclose(out, want)


def small_model(seed=3):
    r = np.random.default_rng(seed)
    cfg = {"input_channels": 2, "num_stems": 3, "channels": [8, 16], "kernel_size": 8,
           "stride": 4, "num_groups": 4}
    chans = [2] + cfg["channels"]
    P = {}
    for i in range(2):
        ci, co = chans[i], chans[i + 1]
        P[f"time_encoder.{i}"] = {"conv.weight": r.standard_normal((co, ci, 8)) * 0.3,
                                  "conv.bias": r.standard_normal(co) * 0.1,
                                  "norm.weight": 1 + 0.1 * r.standard_normal(co),
                                  "norm.bias": 0.1 * r.standard_normal(co)}
    for j in range(2):
        i = 1 - j
        ci, co = chans[i + 1], (2 if i == 0 else chans[i])
        P[f"time_decoder.{j}"] = {"conv_transpose.weight": r.standard_normal((2 * ci, co, 8)) * 0.2,
                                  "conv_transpose.bias": r.standard_normal(co) * 0.1,
                                  "norm.weight": 1 + 0.1 * r.standard_normal(co),
                                  "norm.bias": 0.1 * r.standard_normal(co)}
    for h in range(3):
        P[f"output_heads.{h}"] = {"weight": r.standard_normal((2, 2, 1)),
                                  "bias": r.standard_normal(2)}
    return cfg, P


def test_model_zero_network_gives_head_bias():
    cfg, P = small_model()
    for h in range(3):
        P[f"output_heads.{h}"]["weight"] = np.zeros((2, 2, 1))
    y = osep.separate_time(RNG.standard_normal(2 * 100), P, cfg)
    for h in range(3):
        np.testing.assert_allclose(y[h].reshape(100, 2), np.tile(P[f"output_heads.{h}"]["bias"],
                                                                (100, 1)))


def test_model_composes_layer_oracles():
    cfg, P = small_model()
    n = 130
    x = RNG.standard_normal(2 * n)
    lp, rp, Lp = ol.unet_padding(n, 2, 8, 4)
    assert (lp, rp, Lp) == (7, 7, 16 * 9)
    xp = np.zeros((2, Lp))
    xp[:, lp:lp + n] = x.reshape(n, 2).T
    e0 = ol.encoder_block(xp, *P["time_encoder.0"].values(), 2)
    e1 = ol.encoder_block(e0, *P["time_encoder.1"].values(), 4)
    d0 = ol.decoder_block(e1, e1, *P["time_decoder.0"].values(), 4)
    d1 = ol.decoder_block(d0, e0, *P["time_decoder.1"].values(), 2)
    h1 = ol.conv1d(d1, P["output_heads.1"]["weight"], P["output_heads.1"]["bias"])
    np.testing.assert_allclose(osep.separate_time(x, P, cfg)[1],
                               h1[:, lp:lp + n].T.reshape(-1), atol=1e-12)


def test_time_unet_matches_separator_chain():
    """oracle.layers.time_unet (the U-Net alone) against separate_time's independently written
    chain: with num_groups = 2 every level's GroupNorm has 2 groups in both (separate_time's level-0
    min(groups, input channels) rule gives 2 as well), and one stem whose 1x1 head is the identity
    returns the U-Net output itself, cropped and interleaved. The decoder order (deepest first), the
    skip each decoder level takes and the padding are thereby pinned against each other."""
    r = np.random.default_rng(5)
    cfg = {"input_channels": 2, "num_stems": 1, "channels": [8, 16, 32], "kernel_size": 8,
           "stride": 4, "num_groups": 2}
    chans = [2] + cfg["channels"]
    P, enc, dec = {}, [], []
    for i in range(3):
        ci, co = chans[i], chans[i + 1]
        P[f"time_encoder.{i}"] = {"conv.weight": r.standard_normal((co, ci, 8)) * 0.3,
                                  "conv.bias": r.standard_normal(co) * 0.1,
                                  "norm.weight": 1 + 0.1 * r.standard_normal(co),
                                  "norm.bias": 0.1 * r.standard_normal(co)}
        enc.append(P[f"time_encoder.{i}"])
    for j in range(3):
        i = 2 - j
        ci, co = chans[i + 1], chans[i]
        p = {"conv_transpose.weight": r.standard_normal((2 * ci, co, 8)) * 0.2,
             "conv_transpose.bias": r.standard_normal(co) * 0.1,
             "norm.weight": 1 + 0.1 * r.standard_normal(co),
             "norm.bias": 0.1 * r.standard_normal(co)}
        P[f"time_decoder.{j}"] = p
        dec.append({"conv_tr.weight": p["conv_transpose.weight"],
                    "conv_tr.bias": p["conv_transpose.bias"], "norm.weight": p["norm.weight"],
                    "norm.bias": p["norm.bias"], "groups": 2})
    P["output_heads.0"] = {"weight": np.eye(2)[:, :, None], "bias": np.zeros(2)}
    n = 1500
    x = r.standard_normal(n * 2)
    got = osep.separate_time(x, P, cfg)[0]
    lp, _, Lp = ol.unet_padding(n, 3, 8, 4)
    xp = np.zeros((1, 2, Lp))
    xp[0, :, lp:lp + n] = x.reshape(n, 2).T
    u = ol.time_unet(xp, enc, dec, enc_groups=2)[0]
    np.testing.assert_allclose(got, u[:, lp:lp + n].T.reshape(-1), rtol=1e-12, atol=1e-12)
