"""numpy restatement of the STFT / iSTFT of the frequency branch (reference: zkeown/MetalAudio,
Sources/MetalDSP/STFT.swift and FFT.swift).

TEST INFRASTRUCTURE ONLY — see oracle/__init__.py.
"""
from __future__ import annotations

import numpy as np

__all__ = ["window", "frame_count", "stft", "istft", "dft_bruteforce", "effective_floor"]

FLT_MIN = np.float32(1.17549435e-38)


def window(kind: str, N: int) -> np.ndarray:
    """WindowType.coefficient(at:length:) (FFT.swift:266-296): symmetric (denominator N - 1),
    evaluated in float64 and rounded to float32; length 1 gives 1."""
    if N <= 1:
        return np.ones(N, np.float32)
    n = np.arange(N, dtype=np.float64)
    d = N - 1.0
    if kind == "none":
        w = np.ones(N)
    elif kind == "hann":
        w = 0.5 * (1.0 - np.cos(2.0 * np.pi * n / d))
    elif kind == "hamming":
        w = 0.54 - 0.46 * np.cos(2.0 * np.pi * n / d)
    elif kind == "blackman":
        w = 0.42 - 0.5 * np.cos(2.0 * np.pi * n / d) + 0.08 * np.cos(4.0 * np.pi * n / d)
    else:
        raise ValueError(kind)
    return w.astype(np.float32)


def frame_count(n: int, N: int, hop: int) -> int:
    """STFT.stft (STFT.swift:44-49): inputs shorter than N are an error."""
    if n < N:
        raise ValueError("input shorter than the FFT size")
    return (n - N) // hop + 1


def stft(x, N: int, hop: int, kind: str = "hann", onesided: bool = True, dtype=np.float64):
    """Frames of N samples every hop (no centring), times the window, full DFT without scaling
    (STFT.swift:40-80, forwardBatch). x [n] or [B, n] -> complex [B?, frames, bins]."""
    x = np.asarray(x, dtype=dtype)
    w = window(kind, N).astype(dtype)
    F = frame_count(x.shape[-1], N, hop)
    idx = np.arange(F)[:, None] * hop + np.arange(N)[None, :]
    frames = x[..., idx] * w
    X = np.fft.fft(frames, axis=-1)
    return X[..., :N // 2 + 1] if onesided else X


def effective_floor(f: float) -> float:
    """STFT.swift:491-501."""
    if not f >= 1e-10:
        return 1e-6
    return min(f, 0.1)


def istft(X, N: int, hop: int, kind: str = "hann", onesided: bool = True,
          floor: float = 1e-10, dtype=np.float64):
    """STFT.istft (STFT.swift:384-533): real part of each frame's inverse DFT (1/N), times the
    window, overlap-added in frame order; divided by the overlap-added squared window with sums
    below FLT_MIN set to zero and then floored. X complex [B?, frames, bins]."""
    X = np.asarray(X)
    if onesided:  # rebuild the full spectrum: bins N/2+1..N-1 are the conjugate mirror
        full = np.concatenate([X, np.conj(X[..., 1:N // 2][..., ::-1])], axis=-1)
    else:
        full = X
    frames = np.real(np.fft.ifft(full.astype(np.complex128), axis=-1)).astype(dtype)
    w = window(kind, N).astype(dtype)
    F = frames.shape[-2]
    L = (F - 1) * hop + N
    out = np.zeros(frames.shape[:-2] + (L,), dtype=dtype)
    wsum = np.zeros(L, dtype=dtype)
    for f in range(F):
        out[..., f * hop:f * hop + N] += frames[..., f, :] * w
        wsum[f * hop:f * hop + N] += w * w
    wsum = np.where(wsum < FLT_MIN, 0.0, wsum)
    wsum = np.maximum(wsum, effective_floor(floor))
    return out / wsum


def dft_bruteforce(x):
    """X[k] = sum_n x[n] e^{-2 pi i k n / N} by the definition (small N only)."""
    x = np.asarray(x, dtype=np.complex128)
    N = x.shape[-1]
    k = np.arange(N)
    return x @ np.exp(-2j * np.pi * np.outer(k, k) / N)
