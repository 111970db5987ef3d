"""GPU parity of the configuration table's decoder and frequency-branch rows at the exact sizes
bench.py times them (one 7.8 s chunk, batch 1): the four time-branch UNetDecoderBlock levels at
the config-4 lengths (1344 -> 86016 input samples), the four FreqUNetEncoderBlock2D levels on the
2064 x 336 spectrogram (2 -> 48 -> 96 -> 192 -> 384 channels) and the four mirrored
FreqUNetDecoderBlock2D levels with their skips. The workloads come from bench.py's own setup
functions (same seeds, shapes and weights), and every level is checked against the fp64 oracle
fed with the GPU's own input to that level, so the bar applies per layer and errors do not
compound. At these sizes the kernels take their production forms (K-split GEMMs with the reduce
writing the GroupNorm partials, the implicit-GEMM 2-D conv, the in-place tap GEMM, the few-channel
kernels), which the smaller cases elsewhere reach only one at a time.

fp32 bar: |gpu - oracle| <= 1e-4 + 1e-3 * |oracle| per element."""
import sys

import numpy as np
import pytest

import bench
import oracle
from metalaudio_amd import nn
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


def test_time_decoder_row_full_size(dev, stream):
    dec = bench.decoder_setup(nn, dev)
    y = dec["x"]
    for lvl, (blk, sk, out, p) in enumerate(zip(dec["blocks"], dec["skips"], dec["outs"],
                                                 dec["params"])):
        w, b, gm, bt, g, skh = p
        say(f"time decoder level {lvl}: input {tuple(y.shape)}, skip {skh.shape} -> "
            f"{tuple(out.shape)}, {g} groups")
        blk.forward(y, sk, out, stream)
        stream.sync(60000)
        xin = y.to_numpy()
        ref = oracle.decoder_block(xin, skh, w, b, gm, bt, g)
        assert_close(out.to_numpy(), ref, ATOL, RTOL, f"time decoder level {lvl}")
        y = out


def test_freq_encoder_row_full_size(dev, stream):
    enc, _ = bench.freq_setup(nn, dev)
    y = enc["x"]
    for lvl, (blk, out, p) in enumerate(zip(enc["blocks"], enc["outs"], enc["params"])):
        w, b, gm, bt, g = p
        say(f"frequency encoder level {lvl}: input {tuple(y.shape)} -> {tuple(out.shape)}, "
            f"{g} groups")
        blk.forward(y, out, stream)
        stream.sync(60000)
        ref = oracle.freq_encoder_block(y.to_numpy(), w, b, gm, bt, g)
        assert_close(out.to_numpy(), ref, ATOL, RTOL, f"frequency encoder level {lvl}")
        y = out


def test_freq_decoder_row_full_size(dev, stream):
    _, dec = bench.freq_setup(nn, dev)
    y = dec["x"]
    for lvl, (blk, sk, out, p) in enumerate(zip(dec["blocks"], dec["skips"], dec["outs"],
                                                 dec["params"])):
        w, b, gm, bt, g, skh = p
        say(f"frequency decoder level {lvl}: input {tuple(y.shape)}, skip {skh.shape} -> "
            f"{tuple(out.shape)}, {g} groups")
        blk.forward(y, sk, out, stream)
        stream.sync(60000)
        ref = oracle.freq_decoder_block(y.to_numpy(), skh, w, b, gm, bt, g)
        assert_close(out.to_numpy(), ref, ATOL, RTOL, f"frequency decoder level {lvl}")
        y = out


def test_long_audio_row_full_size(dev, stream):
    """The long-audio row: 60 s of stereo audio through the reference's default time-domain
    HTDemucs (5 levels, 48..768 channels) in 30 s segments with 2 s overlap, as bench.py times it,
    against the fp64 oracle's segmentation and blend (oracle/separate.py) over the whole run."""
    from oracle import separate as osep
    r11, cfg, P = bench.long_audio_setup()
    n = 44100 * 60
    x = r11.uniform(-1, 1, 2 * n).astype(np.float32)
    say(f"long audio: 2 x {n} samples, segments {44100 * 30}, overlap {44100 * 2}")
    sep = nn.Separator(dev)
    sep.load_state(P)
    out = sep.separate_long(nn.Tensor.from_numpy(dev, x), 44100 * 30, 44100 * 2, stream)
    stream.sync(60000)
    ref = osep.separate_long(x, 2, 44100 * 30, 44100 * 2, lambda s: osep.separate_time(s, P, cfg))
    assert out.shape == ref.shape == (4, 2 * n)
    assert_close(out.to_numpy(), ref, ATOL, RTOL, "long audio 60 s")
