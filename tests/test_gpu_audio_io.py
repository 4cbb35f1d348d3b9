"""GPU parity of libstems' separate() data path (stx_separate_audio, audio_io.hip) against the
oracle composed the same way (src/libstems.cpp:135-196).

The model is a per-stem gain (stems[s] = audio * g[s], float32), so every step around it is
checked exactly: the de-interleave and channel mapping and the length pinning are bit-exact; the
resampling both ways is bit-exact with the per-tap kernel (STX_RESAMPLE_EXACT=1) and within the
phase-table kernel's bound (SNR >= 110 dB, every sample within 1e-6 of the rms) by default.
Cases: interleaved and planar, mono / stereo / 3-channel input to a stereo model, equal rates (no
resampling), back-resampled lengths one longer and one shorter than the input (cut and zero
padding), and 6 stems x 2 channels (12 planes: the resampler's 8-plane groups). Errors: the
reference's request checks, plans of the wrong rates, and a model status returned as it is.
"""
import ctypes

import numpy as np
import pytest

import oracle_lib
import stx
import synth
from hip_util import d2d
from metrics import snr_db

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rs():
    return oracle_lib.resample()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def gain_model(gains, device):
    """Model separate: stems[s][c][i] = audio[c][i] * gains[s] on the device, and its oracle."""
    import torch
    g = torch.tensor(gains, dtype=torch.float32, device=device)
    seen = {}

    def sep(audio, channels, length, opt, stems, stream):
        o = ctypes.cast(opt, ctypes.POINTER(stx.SeparateOptions)).contents
        seen.update(channels=channels, length=length, shifts=o.shifts, seed=o.seed)
        a = torch.empty((channels, length), dtype=torch.float32, device=device)
        d2d(a.data_ptr(), audio, channels * length * 4, stream)
        y = (g[:, None, None] * a[None]).contiguous()
        d2d(stems, y.data_ptr(), y.numel() * 4, stream)
        torch.cuda.synchronize()
        return 0

    def oracle(a):
        return np.asarray(gains, np.float32)[:, None, None] * a[None]

    return sep, oracle, seen


def run(device, x, ch, layout, sr, R, gains, monkeypatch=None, **kw):
    import torch
    xd = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32).reshape(-1)).to(device)
    sep, oracle, seen = gain_model(gains, device)
    to_m = stx.Resampler(sr, R) if sr != R else None
    from_m = stx.Resampler(R, sr) if sr != R else None
    out = stx.separate_audio(xd, ch, sr, layout, 2, R, len(gains), sep, to_model=to_m, from_model=from_m, **kw)
    return host(out), oracle, seen


CASES = [  # (input channels, layout, input rate, samples); the model is stereo at 44.1 kHz
    (2, stx.AUDIO_INTERLEAVED, 48000, 1003),     # back-resampled to 1004: cut
    (2, stx.AUDIO_INTERLEAVED, 48000, 1028),     # back-resampled to 1027: zero padding
    (2, stx.AUDIO_PLANAR, 48000, 48000),         # back == n: the resampler writes out itself
    (1, stx.AUDIO_PLANAR, 22050, 30001),         # mono to stereo
    (3, stx.AUDIO_INTERLEAVED, 96000, 1000),     # 3 channels: the first two; back 999
    (2, stx.AUDIO_PLANAR, 44100, 50000),         # planar stereo at the model's rate: no copies
    (3, stx.AUDIO_PLANAR, 44100, 4097),          # equal rates, channel mapping only
    (1, stx.AUDIO_INTERLEAVED, 44100, 1),        # one sample
]


@pytest.mark.parametrize("ch,layout,sr,n", CASES)
def test_separate_audio_bit_exact(device, rs, ch, layout, sr, n, monkeypatch):
    monkeypatch.setenv("STX_RESAMPLE_EXACT", "1")
    gains = [0.5, -1.25, 2.0, 1.0]
    x = synth.normal(n % 997 + ch, (ch * n,), 0.3)
    got, oracle, seen = run(device, x, ch, layout, sr, 44100, gains, shifts=2, seed=7)
    want = rs.separate_audio(x, n, ch, layout, sr, 2, 44100, oracle)
    assert got.shape == (len(gains), 2, n)
    assert np.array_equal(got, want)
    assert seen["channels"] == 2 and seen["length"] == rs.L.orc_resample_length(n, sr, 44100)
    assert seen["shifts"] == 2 and seen["seed"] == 7                  # the request's options reach the model


def test_separate_audio_twelve_planes_default_resampler(device, rs):
    """6 stems x 2 channels (two resampler launches of 8 and 4 planes), the default phase-table
    resampler: SNR >= 110 dB and every sample within 1e-6 of the stems' rms."""
    n, sr = 96000 * 2 + 3, 96000
    gains = [0.5, -1.0, 0.25, 2.0, -0.75, 1.5]
    x = synth.sines_plus_pink(11, 2, n)
    got, oracle, _ = run(device, x, 2, stx.AUDIO_PLANAR, sr, 44100, gains)
    want = rs.separate_audio(x, n, 2, stx.AUDIO_PLANAR, sr, 2, 44100, oracle)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert snr_db(got, want) >= 110.0
    assert float(np.max(np.abs(got.astype(np.float64) - want))) <= 1e-6 * rms


def test_separate_audio_errors(device):
    import torch
    x = torch.zeros(2 * 100, dtype=torch.float32, device=device)
    sep, _, _ = gain_model([1.0], device)
    r = stx.Resampler(48000, 44100)
    cases = [
        dict(shifts=11),                                    # shifts must be 0..10
        dict(overlap=1.0),                                  # overlap must be < 1
        dict(to_model=None),                                # rates differ, no plan
        dict(to_model=r, from_model=r),                     # from_model of the wrong direction
    ]
    for kw in cases:
        args = dict(to_model=r, from_model=stx.Resampler(44100, 48000))
        args.update(kw)
        with pytest.raises(stx.StxError) as e:
            stx.separate_audio(x, 2, 48000, stx.AUDIO_INTERLEAVED, 2, 44100, 1, sep, **args)
        assert e.value.status == stx.STATUS_INVALID_ARGUMENT, kw
    with pytest.raises(stx.StxError) as e:                  # an unknown layout
        stx.separate_audio(x, 2, 44100, 5, 2, 44100, 1, sep)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT and "layout" in e.value.message
    with pytest.raises(stx.StxError) as e:                  # the model's status comes back as it is
        stx.separate_audio(x, 2, 44100, stx.AUDIO_PLANAR, 2, 44100, 1, lambda *a: stx.STATUS_CANCELLED)
    assert e.value.status == stx.STATUS_CANCELLED
