"""Pins of the STFT oracle (oracle/dsp.py) and the host side of the STFT plan: window closed
forms (FFTTests.swift:285-318, 746-800), numpy's FFT against the DFT by definition, frame counts
and output lengths (FFTTests.swift:913-1040), perfect reconstruction where the squared Hann
window overlap-adds above the floor (testSTFTRoundTrip, :1040-1085), and the floor rule."""
import numpy as np
import pytest

from oracle import dsp

RNG = np.random.default_rng(51)


@pytest.mark.parametrize("N", [4, 8, 64, 1024, 4096])
def test_window_closed_forms(N):
    hann = dsp.window("hann", N)
    assert hann[0] == 0 and abs(hann[-1]) < 1e-7 and np.allclose(hann, hann[::-1], atol=1e-6)
    if N % 2:
        assert abs(hann[N // 2] - 1) < 1e-6
    ham = dsp.window("hamming", N)
    assert abs(ham[0] - 0.08) < 1e-6 and np.allclose(ham, ham[::-1], atol=1e-6)
    bl = dsp.window("blackman", N)
    assert abs(bl[0]) < 1e-6 and bl.max() <= 1.0 + 1e-6
    assert np.all(dsp.window("none", N) == 1)
    n = np.arange(N)
    np.testing.assert_allclose(hann, 0.5 - 0.5 * np.cos(2 * np.pi * n / (N - 1)), atol=1e-7)


def test_fft_matches_definition():
    for N in (4, 8, 16, 128):
        x = RNG.standard_normal((3, N))
        np.testing.assert_allclose(np.fft.fft(x), dsp.dft_bruteforce(x), atol=1e-9)


def test_stft_frames_and_spectrum_by_definition():
    N, hop = 16, 4
    x = RNG.standard_normal(70)
    X = dsp.stft(x, N, hop, onesided=False)
    assert X.shape == (dsp.frame_count(70, N, hop), N) == ((70 - 16) // 4 + 1, 16)
    w = dsp.window("hann", N)
    for f in (0, 5, X.shape[0] - 1):
        np.testing.assert_allclose(X[f], dsp.dft_bruteforce(x[f * hop:f * hop + N] * w),
                                   atol=1e-9)
    Xh = dsp.stft(x, N, hop)
    np.testing.assert_allclose(Xh, X[:, :N // 2 + 1])
    # real input: Hermitian spectrum
    np.testing.assert_allclose(X[:, 1:][:, ::-1], np.conj(X[:, 1:]), atol=1e-9)
    with pytest.raises(ValueError):
        dsp.stft(x[:15], N, hop)


@pytest.mark.parametrize("N,hop,kind", [(16, 4, "hann"), (64, 16, "hann"), (64, 32, "hamming"),
                                        (128, 32, "blackman"), (32, 8, "none")])
def test_round_trip_reconstructs_where_window_covers(N, hop, kind):
    x = RNG.standard_normal(N * 6 + 3)
    X = dsp.stft(x, N, hop, kind)
    y = dsp.istft(X, N, hop, kind)
    L = len(y)
    assert L == (X.shape[0] - 1) * hop + N
    w2 = np.zeros(L)
    w = dsp.window(kind, N).astype(np.float64)
    for f in range(X.shape[0]):
        w2[f * hop:f * hop + N] += w * w
    ok = w2 > 1e-3
    np.testing.assert_allclose(y[ok], x[:L][ok], atol=1e-9)


def test_floor_rule():
    assert dsp.effective_floor(1e-10) == 1e-10
    assert dsp.effective_floor(1e-11) == 1e-6
    assert dsp.effective_floor(0.5) == 0.1
    assert dsp.effective_floor(1e-3) == 1e-3
