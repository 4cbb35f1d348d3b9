"""CPU checks that pin the TFC-TDF chunking oracle (oracle/tfc_oracle.c).

No reference test covers demix_msst / demix_uvr (the reference's fixtures need the models).
Pins: a numpy float32 restatement of the reference's linspace for the MSST fades (and
torch.linspace, which it imitates, to one ulp), numpy's np.hanning for the UVR weights, independent numpy restatements of both loops (bit for bit: the
same float/double operations in the same order), the UVR geometry of the defaults, and the
identity model, which both loops must return unchanged.
"""
import numpy as np
import pytest

import oracle_lib
import synth


@pytest.fixture(scope="module")
def od():
    return oracle_lib.demix()


def np_linspace(a, b, n):
    """linspace of src/tfc_tdf.cpp:55-63 in numpy float32: a + step * i for the first half, b -
    step * (n - 1 - i) for the second."""
    v = np.zeros(max(n, 0), np.float32)
    if n == 1:
        v[0] = a
    if n < 2:
        return v
    a, b = np.float32(a), np.float32(b)
    step = (b - a) / np.float32(n - 1)
    for i in range(n):
        v[i] = a + step * np.float32(i) if i < n // 2 else b - step * np.float32(n - 1 - i)
    return v


def msst_window_np(chunk):
    fade = chunk // 10
    w = np.ones(chunk, np.float32)
    if fade > 0:
        w[:fade] = np_linspace(0, 1, fade)
        w[chunk - fade:] = np_linspace(1, 0, fade)
    return w


@pytest.mark.parametrize("chunk", [100, 101, 9, 10, 19, 261120])
def test_msst_window(od, chunk):
    """The reference's own linspace, and torch.linspace (which it imitates) to one float ulp: torch
    2.10's CPU kernel rounds a few points of the second half the other way."""
    import torch
    w = od.msst_window(chunk)
    assert np.array_equal(w, msst_window_np(chunk))
    fade = chunk // 10
    if fade > 1:
        t = torch.linspace(0, 1, fade, dtype=torch.float32).numpy()
        assert np.max(np.abs(w[:fade] - t)) <= 6e-8 and w[0] == 0.0 and w[fade - 1] == 1.0
        assert w[chunk - fade] == 1.0 and w[chunk - 1] == 0.0


def np_reflect(x, left, right):
    return np.pad(x.astype(np.float64), (left, right), mode="reflect").astype(np.float32)


def np_msst(mix, chunk, step, model):
    """demix_msst (src/tfc_tdf.cpp:447-495) restated in numpy."""
    C, L = mix.shape
    border = chunk - step
    pad = L > 2 * border and border > 0
    x = np.stack([np_reflect(m, border, border) for m in mix]) if pad else mix.copy()
    Lp = x.shape[1]
    fade = chunk // 10
    window = msst_window_np(chunk)
    result, counter = None, np.zeros(Lp)
    i = 0
    while i < Lp:
        n = min(chunk, Lp - i)
        part = np.zeros((C, chunk), np.float32)
        part[:, :n] = x[:, i:i + n]
        if n < chunk:
            part = np.stack([np_reflect(p[:n], 0, chunk - n) for p in part]) if n > chunk // 2 else part
        y = model(part)                                           # [S][C][chunk]
        if result is None:
            result = np.zeros((y.shape[0], C, Lp))
        w = window.copy()
        if i == 0:
            w[:fade] = 1.0
        elif i + step >= Lp:
            w[chunk - fade:] = 1.0
        result[:, :, i:i + n] += y[:, :, :n].astype(np.float64) * w[:n].astype(np.float64)
        counter[i:i + n] += w[:n]
        i += step
    off = border if pad else 0
    v = result[:, :, off:off + L] / counter[off:off + L]
    return np.where(np.isfinite(v), v, 0.0).astype(np.float32)


@pytest.mark.parametrize("L,chunk,step", [(1000, 100, 25), (1000, 100, 100), (150, 100, 25), (1001, 97, 31),
                                          (60, 100, 50), (5003, 64, 9)])
def test_msst_vs_numpy(od, L, chunk, step):
    mix = synth.normal(L, (2, L), 0.5)
    g = np.array([0.5, -2.0], np.float32)[:, None, None]
    parts = od.msst_chunks(mix, chunk, step)
    got = od.msst_ola(g[None] * parts[:, None], L, chunk, step)
    assert np.array_equal(got, np_msst(mix, chunk, step, lambda p: g * p[None]))


def test_msst_differs_from_roformer_where_the_reference_does(od):
    """A short chunk of exactly chunk/2 + 1 samples: MSST reflect-pads it, RoFormer zero-pads."""
    chunk, step = 100, 100
    L = 3 * chunk + chunk // 2 + 1                  # no border pad (border 0); last chunk 51 samples
    mix = synth.normal(2, (1, L), 1.0)
    m = od.msst_chunks(mix, chunk, step)[-1, 0]
    r = od.chunks(mix, chunk, step)[-1, 0]
    assert np.all(r[51:] == 0.0) and not np.all(m[51:] == 0.0)


def np_uvr(mix, chunk, n_fft, overlap, model):
    """demix_uvr (src/tfc_tdf.cpp:407-441) restated in numpy."""
    C, L = mix.shape
    trim, gen = n_fft // 2, chunk - n_fft
    M = trim + L + gen + trim - L % gen
    step = chunk - n_fft if overlap < 0 else int((1.0 - overlap) * chunk)
    x = np.zeros((C, M), np.float32)
    x[:, trim:trim + L] = mix
    result, div = None, np.zeros(M)
    for i in range(0, M, step):
        actual = min(chunk, M - i)
        part = np.zeros((C, chunk), np.float32)
        part[:, :actual] = x[:, i:i + actual]
        y = model(part)
        if result is None:
            result = np.zeros((y.shape[0], C, M))
        w = np.ones(actual) if overlap == 0 else np.hanning(actual)
        result[:, :, i:i + actual] += y[:, :, :actual].astype(np.float64) * w
        div[i:i + actual] += w
    return (result[:, :, trim:trim + L] / div[trim:trim + L]).astype(np.float32)


@pytest.mark.parametrize("L,chunk,n_fft,overlap", [(5000, 512, 128, -1.0), (5000, 512, 128, 0.5), (5000, 512, 128, 0.0),
                                                   (300, 512, 128, -1.0), (4099, 600, 100, 0.25)])
def test_uvr_vs_numpy(od, L, chunk, n_fft, overlap):
    mix = synth.normal(L + chunk, (2, L), 0.5)
    g = np.array([1.5, -0.25, 3.0], np.float32)[:, None, None]
    parts = od.uvr_chunks(mix, chunk, n_fft, overlap)
    got = od.uvr_ola(g[None] * parts[:, None], L, chunk, n_fft, overlap)
    want = np_uvr(mix, chunk, n_fft, overlap, lambda p: g * p[None])
    # np.hanning evaluates cos at (pi n / (M-1)) from the centre; the reference (and the
    # oracle) at 2 pi i / (M-1) from the start: the weights agree to ~1e-16, not bit for bit.
    assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))
    if overlap == 0.0:
        assert np.array_equal(got, want)


def test_uvr_geometry_defaults(od):
    """Kim_Vocal_2-like: n_fft 7680, hop 1024, dim_t 256 -> chunk 1024 * 255 = 261,120."""
    n, M, step = od.uvr_geometry(7938000, 261120, 7680)
    gen = 261120 - 7680
    assert step == gen and M == 3840 + 7938000 + gen + 3840 - 7938000 % gen and n == -(-M // step)
    assert od.uvr_geometry(100, 100, 128)[0] == -1                # chunk shorter than the FFT
    assert od.uvr_geometry(1000, 512, 128, 1.0)[0] == -2          # overlap too large


def test_identity_models(od):
    mix = synth.normal(9, (2, 7000), 0.5)
    ident = lambda p: p[None]
    u = od.uvr_ola(od.uvr_chunks(mix, 1024, 256, 0.5)[:, None], 7000, 1024, 256, 0.5)[0]
    m = od.msst_ola(od.msst_chunks(mix, 1000, 250)[:, None], 7000, 1000, 250)[0]
    assert np.max(np.abs(u - mix)) <= 2e-7 * np.max(np.abs(mix))
    assert np.max(np.abs(m - mix)) <= 2e-7 * np.max(np.abs(mix))


def test_tfc_post(od):
    mix = synth.normal(10, (2, 50), 1.0)
    est = synth.normal(11, (2, 2, 50), 1.0)
    out = od.tfc_post(mix, est, 1.035, True)
    comp = est * np.float32(1.035)
    assert np.array_equal(out[:2], comp)
    assert np.array_equal(out[2], (mix - comp[0]) - comp[1])
