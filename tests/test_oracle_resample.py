"""CPU checks that pin the resampler oracle (oracle/resample_oracle.c, src/audio.h:17-59).

No reference test covers resample_planar. Pins: equal rates return the input; a numpy
restatement of the tabulated kernel (same double operations, bit for bit); the untabulated
Kaiser-sinc formula (to the table's linear-interpolation error); and closed forms: a sine well
inside the passband keeps its amplitude and phase, and DC stays DC.
"""
import numpy as np
import pytest

import oracle_lib
import synth


@pytest.fixture(scope="module")
def rs():
    return oracle_lib.resample()


def np_resample(x, src, dst, table, half):
    ratio = dst / src
    C, n = x.shape
    out_n = int(np.rint(n * ratio)) if (n * ratio) % 1 != 0.5 else int(np.floor(n * ratio + 0.5))
    tn = 1 << 15
    out = np.zeros((C, out_n), np.float32)
    for i in range(out_n):
        c = i / ratio
        lo, hi = max(0, int(np.ceil(c - half))), min(n - 1, int(np.floor(c + half)))
        acc = np.zeros(C)
        for j in range(lo, hi + 1):
            pos = abs(j - c) / half * tn
            t = int(pos)
            if t >= tn:
                continue
            fr = pos - t
            w = table[t] + (table[t + 1] - table[t]) * fr
            acc += w * x[:, j].astype(np.float64)
        out[:, i] = acc.astype(np.float32)
    return out


def test_equal_rates_identity(rs):
    x = synth.normal(1, (2, 100), 1.0)
    assert np.array_equal(rs(x, 44100, 44100), x)


@pytest.mark.parametrize("src,dst", [(48000, 44100), (22050, 44100), (44100, 16000)])
def test_vs_numpy_and_formula(rs, src, dst):
    x = synth.normal(src % 97, (2, 400), 1.0)
    table, half = rs.table(src, dst)
    got = rs(x, src, dst)
    assert np.array_equal(got, np_resample(x, src, dst, table, half))
    # The table is the Kaiser-windowed sinc it claims to be.
    from scipy.special import i0
    ratio = dst / src
    cutoff = 0.95 * min(1.0, ratio)
    xs = np.arange(0, (1 << 15) + 2) / (1 << 15)
    xs = np.minimum(xs, 1.0) * half
    r = xs / half
    want = np.where(r >= 1, 0.0, np.sinc(xs * cutoff) * i0(8.6 * np.sqrt(np.maximum(1 - r * r, 0))) / i0(8.6) * cutoff)
    assert np.max(np.abs(table - want)) <= 1e-12


def test_passband_sine_and_dc(rs):
    src, dst, n = 48000, 44100, 48000
    t = np.arange(n) / src
    x = np.stack([np.sin(2 * np.pi * 1000 * t), np.ones(n)]).astype(np.float32)
    y = rs(x, src, dst)
    m = y.shape[1]
    ty = np.arange(m) / dst
    mid = slice(200, m - 200)
    assert np.max(np.abs(y[0, mid] - np.sin(2 * np.pi * 1000 * ty[mid]))) <= 2e-3
    assert np.max(np.abs(y[1, mid] - 1.0)) <= 2e-3


@pytest.mark.parametrize("ch,layout,want", [(2, 0, 2), (2, 1, 2), (1, 0, 2), (1, 1, 2), (3, 1, 2), (3, 0, 2),
                                             (2, 1, 1), (4, 1, 6)])
def test_to_channels_against_numpy(rs, ch, layout, want):
    """libstems' de-interleave (src/libstems.cpp:160-167) and st::to_channels (src/audio.h:62-71)
    against numpy's transpose and a fancy index by the channel map."""
    n = 37
    x = synth.normal(ch * 10 + layout, (ch * n,), 1.0).astype(np.float32)
    planar = x.reshape(n, ch).T if layout == 1 else x.reshape(ch, n)
    src = list(range(want)) if ch == want else [0 if ch == 1 else min(c, ch - 1) for c in range(want)]
    assert np.array_equal(rs.to_channels(x, n, ch, layout, want), planar[src])


@pytest.mark.parametrize("back,n", [(10, 10), (12, 10), (7, 10), (1, 3)])
def test_pin_length_against_numpy(rs, back, n):
    """The length pinning of src/libstems.cpp:188-193: cut to n, or padded with zeros."""
    x = synth.normal(back + n, (3, back), 1.0).astype(np.float32)
    want = np.zeros((3, n), np.float32)
    m = min(back, n)
    want[:, :m] = x[:, :m]
    assert np.array_equal(rs.pin_length(x, n), want)
