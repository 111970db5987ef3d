"""GPU parity of the STFT / iSTFT kernels (STFT.swift:40-533) through the C ABI against the fp64
oracle (oracle/dsp.py): spectra in both layouts, onesided and full, batched; the inverse from
onesided and from full (non-Hermitian) spectra; the round trip; the HTDemucs size (nfft 4096,
hop 1024) on a 7.8 s stereo chunk.

Tolerance: an fp32 FFT's error grows with the transform's norm, so spectra are compared as
max |gpu - oracle| <= 2e-6 * max |oracle| (measured ~1e-7); time signals per element at
abs 1e-4 + rel 1e-3 where the squared window overlap-adds above 1e-3, and, against the oracle's
inverse of the same spectra, within 1e-3 of the output's scale elsewhere (there the floor
division amplifies the rounding)."""
import sys

import numpy as np
import pytest

from metalaudio_amd import nn
from oracle import dsp

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(61)


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    return nn.AudioDevice(0)


@pytest.fixture(scope="module")
def stream(dev):
    return nn.Stream(dev)


def spec_close(got, ref, what):
    err = float(np.abs(got - ref).max())
    scale = float(np.abs(ref).max())
    assert np.all(np.isfinite(got)) and err <= 2e-6 * scale, \
        f"{what}: max abs {err:.3e} vs 2e-6 * {scale:.3e}"


@pytest.mark.parametrize("N,hop,kind,B,n", [
    (4, 1, "hann", 1, 37), (8, 2, "hamming", 2, 100), (64, 16, "hann", 1, 1000),
    # the register-resident FFT's sizes: 16 frames per workgroup, 90 frames (ragged) and 64
    (128, 32, "hann", 2, 3000), (256, 64, "hamming", 1, 4288), (2048, 512, "hann", 1, 22016),
    (512, 128, "blackman", 3, 5000), (1024, 256, "none", 1, 4096), (4096, 1024, "hann", 2, 50000),
    (8192, 2048, "hann", 1, 30000),  # largest size with the twiddle table staged in LDS
    (16384, 4096, "hann", 1, 40000),
    (4096, 1024, "hann", 2, 343980),  # a 7.8 s stereo chunk: 332 frames, whole 4-frame vectors
])
@pytest.mark.parametrize("onesided,layout", [(True, "frames"), (False, "frames"), (True, "bins"),
                                             (False, "bins")])
def test_stft_forward_parity(dev, stream, N, hop, kind, B, n, onesided, layout):
    say(f"stft N={N} hop={hop} {kind} B={B} n={n} onesided={onesided} layout={layout}")
    x = RNG.standard_normal((B, n)).astype(np.float32)
    plan = nn.STFT(dev, N, hop, kind)
    re, im = plan.stft(nn.Tensor.from_numpy(dev, x), onesided, layout, stream)
    stream.sync(60000)
    ref = dsp.stft(x, N, hop, kind, onesided)
    if layout == "bins":
        ref = np.swapaxes(ref, -1, -2)
    got = re.to_numpy() + 1j * im.to_numpy()
    assert got.shape == ref.shape
    spec_close(got, ref, "spectrum")


def signal_close(got, ref, wsum, what, edges=True):
    ok = wsum > 1e-3
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got))
    assert np.all(err[..., ok] <= 1e-4 + 1e-3 * np.abs(ref[..., ok])), \
        f"{what}: max err {err[..., ok].max():.3e} where the window covers"
    if edges:
        assert err.max() <= 1e-3 * max(1.0, float(np.abs(ref).max())), what


def wsum_of(N, hop, kind, F):
    w = dsp.window(kind, N).astype(np.float64)
    s = np.zeros((F - 1) * hop + N)
    for f in range(F):
        s[f * hop:f * hop + N] += w * w
    return s


@pytest.mark.parametrize("N,hop,kind,B,F", [(4, 1, "hann", 1, 13), (8, 2, "hann", 1, 9),
                                            (128, 32, "hann", 1, 45), (256, 64, "hann", 2, 32),
                                            (2048, 512, "blackman", 1, 16),
                                            (64, 16, "hann", 2, 40),
                                            (512, 256, "hamming", 1, 30),
                                            (4096, 1024, "hann", 2, 20),
                                            (4096, 1024, "hann", 2, 23),
                                            # twiddles in LDS at its limit, then from global memory
                                            (8192, 2048, "hann", 1, 9),
                                            (16384, 4096, "hann", 1, 7)])
@pytest.mark.parametrize("onesided,layout", [(True, "frames"), (False, "frames"), (True, "bins"),
                                             (False, "bins")])
def test_istft_parity(dev, stream, N, hop, kind, B, F, onesided, layout):
    say(f"istft N={N} hop={hop} {kind} B={B} F={F} onesided={onesided} layout={layout}")
    bins = N // 2 + 1 if onesided else N
    # arbitrary spectra (the full one not Hermitian): the inverse keeps the real part
    X = (RNG.standard_normal((B, F, bins)) + 1j * RNG.standard_normal((B, F, bins))) * 10
    X = X.astype(np.complex64)
    ref = dsp.istft(X, N, hop, kind, onesided)
    Xl = np.swapaxes(X, -1, -2) if layout == "bins" else X
    plan = nn.STFT(dev, N, hop, kind)
    y = plan.istft(nn.Tensor.from_numpy(dev, np.ascontiguousarray(Xl.real)),
                   nn.Tensor.from_numpy(dev, np.ascontiguousarray(Xl.imag)), onesided, layout,
                   stream=stream)
    stream.sync(60000)
    signal_close(y.to_numpy(), ref, wsum_of(N, hop, kind, F), "istft")


def test_round_trip_htdemucs_chunk(dev, stream):
    """nfft 4096, hop 1024 (HTDemucs.swift:47-48) on a stereo 7.8 s chunk: the spectrogram and
    the reconstruction."""
    n = 343980
    say(f"round trip 2 x {n} samples, nfft 4096 hop 1024")
    x = RNG.uniform(-1, 1, (2, n)).astype(np.float32)
    plan = nn.STFT(dev, 4096, 1024, "hann")
    xt = nn.Tensor.from_numpy(dev, x)
    re, im = plan.stft(xt, True, "bins", stream)
    y = plan.istft(re, im, True, "bins", stream=stream)
    stream.sync(60000)
    ref = dsp.stft(x, 4096, 1024)
    spec_close(re.to_numpy() + 1j * im.to_numpy(), np.swapaxes(ref, -1, -2), "spectrogram")
    L = y.shape[-1]
    # Against the input itself only where the squared window overlap-adds above 1e-3: in the
    # first and last samples the division by a near-zero window sum (STFT.swift:503-531)
    # amplifies any rounding of the frames, in the reference's fp32 as here.
    signal_close(y.to_numpy(), x[:, :L].astype(np.float64),
                 wsum_of(4096, 1024, "hann", ref.shape[-2]), "round trip", edges=False)


def test_plan_tables_and_shapes(dev):
    p = nn.STFT(dev, 64, 16, "hann")
    np.testing.assert_array_equal(p.window, dsp.window("hann", 64))
    for kind in ("none", "hamming", "blackman"):
        np.testing.assert_array_equal(nn.STFT(dev, 32, 8, kind).window, dsp.window(kind, 32))
    assert p.frame_count(1000) == dsp.frame_count(1000, 64, 16)
    assert p.output_length(10) == 9 * 16 + 64


def test_stft_errors(dev, stream):
    with pytest.raises(nn.MNNError):
        nn.STFT(dev, 1000, 250)  # not a power of 2
    with pytest.raises(nn.MNNError):
        nn.STFT(dev, 32768, 1024)  # above the LDS transform's limit
    plan = nn.STFT(dev, 64, 16)
    with pytest.raises(nn.MNNError):
        plan.frame_count(63)
    with pytest.raises(nn.MNNError):
        plan.stft(nn.Tensor.from_numpy(dev, np.zeros(63, np.float32)), stream=stream)
    re = nn.Tensor(dev, (4, 30))
    with pytest.raises(nn.MNNError):  # 30 bins is neither 33 nor 64
        plan.istft(re, re, stream=stream)
