"""Seeded synthetic inputs shared by the parity tests and the benchmark.

A counter-based generator (splitmix64 of seed and element index) makes every buffer a pure
function of (seed, shape), so the CPU oracle and the GPU consume the same bytes and a buffer
can be regenerated anywhere without state. Normal deviates use Box-Muller in double, then
round to float32.
"""
import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, stream: int = 0) -> np.ndarray:
    """n 64-bit outputs of splitmix64 at counters 1..n from base (seed, stream)."""
    base = np.uint64((seed * 0x632BE59BD9B4E019 + stream * 0xD1B54A32D192ED03) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        z = base + (np.arange(1, n + 1, dtype=np.uint64) * _GAMMA)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, n: int, stream: int = 0) -> np.ndarray:
    """Doubles in [0, 1) with 53 random bits."""
    return (splitmix64(seed, n, stream) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, shape, sigma: float = 1.0, stream: int = 0) -> np.ndarray:
    """float32 N(0, sigma^2) of the given shape."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = uniform01(seed, 2 * m, stream)
    r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
    th = 2.0 * np.pi * u[1::2]
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(th)
    z[1::2] = r * np.sin(th)
    return (sigma * z[:n]).astype(np.float32).reshape(shape)


def uniform(seed: int, shape, lo: float = -1.0, hi: float = 1.0, stream: int = 0) -> np.ndarray:
    """float32 uniform in [lo, hi)."""
    n = int(np.prod(shape))
    return (lo + (hi - lo) * uniform01(seed, n, stream)).astype(np.float32).reshape(shape)


def sines_plus_pink(seed: int, channels: int, n: int, sr: int = 44100, n_sines: int = 8) -> np.ndarray:
    """Sum of seeded sines (f in [40 Hz, 0.4 sr], amp in [0.02, 0.2]) plus seeded pink noise,
    float32 [channels][n]: the full-song test signal."""
    out = np.empty((channels, n), dtype=np.float32)
    t = np.arange(n, dtype=np.float64)
    for c in range(channels):
        p = uniform01(seed, 3 * n_sines, stream=100 + c)
        f = 40.0 + (0.4 * sr - 40.0) * p[0::3]
        ph = 2.0 * np.pi * p[1::3]
        a = 0.02 + 0.18 * p[2::3]
        s = np.zeros(n, dtype=np.float64)
        for k in range(n_sines):
            s += a[k] * np.sin(2.0 * np.pi * f[k] / sr * t + ph[k])
        # Pink noise: white noise shaped by 1/sqrt(f) in the frequency domain.
        w = normal(seed, (n,), 1.0, stream=200 + c).astype(np.float64)
        W = np.fft.rfft(w)
        k = np.arange(W.size, dtype=np.float64)
        k[0] = 1.0
        pink = np.fft.irfft(W / np.sqrt(k), n)
        pink *= 0.05 / max(pink.std(), 1e-12)
        out[c] = (s + pink).astype(np.float32)
    return out
