"""CPU checks that pin the STFT oracle (oracle/stft_oracle.c) before it is trusted.

1. Bit-exact against golden vectors written by the reference's own src/stft.h.
2. Bit-exact against the reference build itself on further sizes, where oracle/_ref exists.
3. Closed forms a plausible mistake would break: brute-force DFT, impulse known answer
   (tests/vr_dsp_test.cpp:8-15 style), Parseval, numpy's rfft on explicitly padded frames.
4. The reference's own round-trip tolerances (tests/dsp_test.cpp:53-96).
"""
import glob
import os

import numpy as np
import pytest

import oracle_lib
import synth

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "stft_*.npz")))


@pytest.fixture(scope="module")
def orc():
    return oracle_lib.oracle()


def test_golden_vectors_present():
    assert len(GOLDEN) >= 15


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[5:-4] for p in GOLDEN])
def test_oracle_matches_reference_golden(orc, path):
    d = np.load(path)
    name = os.path.basename(path)
    if name.startswith("stft_fft_impulse"):
        assert np.array_equal(orc.fft(d["x"]), d["X"])
    elif name.startswith("stft_fft_"):
        assert np.array_equal(orc.fft(d["x"]), d["X"])
        assert np.array_equal(orc.fft(d["X"], True), d["x_back"])
    elif name.startswith("stft_torch"):
        n, h, nm = int(d["n_fft"]), int(d["hop"]), int(d["normalized"])
        assert np.array_equal(orc.torch_stft(d["x"], n, h, nm), d["spec"])
        assert np.array_equal(orc.torch_istft(d["spec"], n, h, nm), d["y"])
    else:
        n = int(d["n_fft"])
        assert np.array_equal(orc.htdemucs_spec(d["x"], n), d["spec"])
        assert np.array_equal(orc.htdemucs_ispec(d["spec"], n, d["x"].size), d["y"])


@pytest.mark.skipif(not oracle_lib.ref_available(), reason="oracle/_ref not built (no /root/reference)")
@pytest.mark.parametrize("n_fft,hop,length", [(1024, 256, 5000), (2048, 441, 441 * 7 + 3), (512, 100, 1025)])
def test_oracle_matches_reference_build(orc, n_fft, hop, length):
    ref = oracle_lib.reference()
    x = synth.normal(77 + n_fft, (length,), 0.3)
    for norm in (False, True):
        s = ref.torch_stft(x, n_fft, hop, norm)
        assert np.array_equal(orc.torch_stft(x, n_fft, hop, norm), s)
        assert np.array_equal(orc.torch_istft(s, n_fft, hop, norm), ref.torch_istft(s, n_fft, hop, norm))
    if length > n_fft:
        s = ref.htdemucs_spec(x, n_fft)
        assert np.array_equal(orc.htdemucs_spec(x, n_fft), s)
        assert np.array_equal(orc.htdemucs_ispec(s, n_fft, length), ref.htdemucs_ispec(s, n_fft, length))


@pytest.mark.parametrize("n", [2, 8, 16, 64, 256])
def test_fft_brute_force(orc, n):
    v = synth.normal(5 + n, (2 * n,), 1.0).astype(np.float64)
    a = v[0::2] + 1j * v[1::2]
    k = np.arange(n)
    W = np.exp(-2j * np.pi * np.outer(k, k) / n)
    assert np.max(np.abs(orc.fft(a) - W @ a)) < 1e-12 * n
    assert np.max(np.abs(orc.fft(a, True) - np.conj(W) @ a)) < 1e-12 * n


@pytest.mark.parametrize("n", [512, 2048, 4096])
def test_fft_impulse_known_answer(orc, n):
    x = np.zeros(n, dtype=np.complex128)
    x[7] = 1.0
    X = orc.fft(x)
    k = np.arange(n)
    assert np.max(np.abs(X - np.exp(-2j * np.pi * 7 * k / n))) < 1e-10
    assert np.max(np.abs(orc.fft(X, True) / n - x)) < 1e-10


def test_fft_round_trip_and_parseval(orc):
    v = synth.uniform(1234, (2 * 4096,), -1.0, 1.0).astype(np.float64)
    a = v[0::2] + 1j * v[1::2]
    X = orc.fft(a)
    assert np.max(np.abs(orc.fft(X, True) / 4096.0 - a)) < 1e-12          # dsp_test.cpp:63
    assert abs(np.sum(np.abs(a) ** 2) - np.sum(np.abs(X) ** 2) / 4096) < 1e-9


def test_fft_rejects_non_power_of_two(orc):
    with pytest.raises(ValueError):
        orc.fft(np.zeros(12, dtype=np.complex128))


def _hann(n):
    return 0.5 - 0.5 * np.cos(2.0 * np.pi * np.arange(n) / n)


@pytest.mark.parametrize("normalized", [False, True])
def test_torch_stft_equals_numpy_rfft(orc, normalized):
    n, hop, length = 256, 64, 1000
    x = synth.normal(9, (length,), 0.1)
    xp = np.pad(x.astype(np.float64), n // 2, mode="reflect")   # torch reflect == numpy reflect
    T = length // hop + 1
    frames = np.stack([xp[t * hop:t * hop + n] * _hann(n) for t in range(T)], axis=1)
    want = np.fft.rfft(frames, axis=0) * (1 / np.sqrt(n) if normalized else 1.0)
    assert np.max(np.abs(orc.torch_stft(x, n, hop, normalized) - want)) < 1e-12


def test_htdemucs_spec_equals_numpy_rfft(orc):
    n, length = 256, 64 * 9 + 5
    hl = n // 4
    x = synth.normal(10, (length,), 0.1)
    le = -(-length // hl)
    pad = hl // 2 * 3
    x1 = np.pad(x.astype(np.float64), (pad, pad + le * hl - length), mode="reflect")
    xp = np.pad(x1, n // 2, mode="reflect")
    frames = np.stack([xp[(t + 2) * hl:(t + 2) * hl + n] * _hann(n) for t in range(le)], axis=1)
    want = np.fft.rfft(frames, axis=0)[: n // 2] / np.sqrt(n)
    assert np.max(np.abs(orc.htdemucs_spec(x, n) - want)) < 1e-12


@pytest.mark.parametrize("normalized", [False, True])
def test_torch_round_trip_reference_tolerance(orc, normalized):
    # tests/dsp_test.cpp:66-78: n_fft 2048, hop 441, len 441*200, max |x - y| < 1e-5.
    n, hop = 2048, 441
    x = synth.uniform(42, (hop * 200,), -1.0, 1.0)
    y = orc.torch_istft(orc.torch_stft(x, n, hop, normalized), n, hop, normalized)
    assert y.size == x.size and np.max(np.abs(x - y)) < 1e-5


def test_htdemucs_round_trip_reference_tolerance(orc):
    # tests/dsp_test.cpp:80-96: band-limited (24 sines below 0.4 sr), 4096/1024, len 1024*60,
    # max |x - y| < 1e-6 more than 4096 samples from either end.
    length, sr = 1024 * 60, 44100
    p = synth.uniform01(7, 72)
    f, ph, amp = 40.0 + (0.4 * sr - 40.0) * p[0::3], 2 * np.pi * p[1::3], 0.02 + 0.18 * p[2::3]
    t = np.arange(length)
    x = sum(amp[k] * np.sin(2 * np.pi * f[k] * t / sr + ph[k]) for k in range(24)).astype(np.float32)
    spec = orc.htdemucs_spec(x, 4096)
    y = orc.htdemucs_ispec(spec, 4096, length)
    assert spec.shape[1] == length // 1024
    assert np.max(np.abs(x[4096:-4096] - y[4096:-4096])) < 1e-6


def test_reflect_pad_errors(orc):
    with pytest.raises(RuntimeError):
        orc.torch_stft(np.zeros(1024, np.float32), 2048, 441)        # len <= n/2
    with pytest.raises(RuntimeError):
        orc.htdemucs_spec(np.zeros(1000, np.float32), 4096)          # len <= pad (1536)


# ----------------------------------------------- st::VRFFT (Bluestein) for other sizes
@pytest.mark.parametrize("n", [7680, 960, 640, 320, 15])
def test_vrfft_is_a_dft(n):
    """orc_vrfft (src/vr_dsp.h:11-37) against the DFT by its definition, in double."""
    o = oracle_lib.oracle()
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    k = np.arange(n)
    if n <= 1000:
        want = np.exp(-2j * np.pi * np.outer(k, k) / n) @ x
    else:
        want = np.fft.fft(x)                                 # pinned to the definition at the small sizes
    got = o.vrfft(x)
    assert np.max(np.abs(got - want)) <= 1e-9 * np.max(np.abs(want))
    back = o.vrfft(got, inverse=True) / n
    assert np.max(np.abs(back - x)) <= 1e-12 * np.max(np.abs(x))


def test_torch_stft_istft_7680_round_trip():
    """torch_stft -> torch_istft with the Kim_Vocal_2 transform (n_fft 7680, hop 1024): the
    identity away from the edges, as the reference's power-of-two round trips
    (tests/dsp_test.cpp:63,76-77)."""
    o = oracle_lib.oracle()
    x = synth.normal(3, (30000,), 0.3)
    spec = o.torch_stft(x, 7680, 1024)
    y = o.torch_istft(spec, 7680, 1024)
    n = min(len(y), len(x))
    assert np.max(np.abs(y[:n] - x[:n])) <= 1e-6 * np.max(np.abs(x))
    # Bin f of frame t is the DFT of the windowed, reflect-padded frame at that bin.
    xp = np.pad(x.astype(np.float64), (3840, 3840), mode="reflect")
    w = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(7680) / 7680)
    t = 7
    frame = xp[t * 1024:t * 1024 + 7680] * w
    assert np.max(np.abs(spec[:, t] - np.fft.rfft(frame))) <= 1e-9 * np.max(np.abs(spec[:, t]))
