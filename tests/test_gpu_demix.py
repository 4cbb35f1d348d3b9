"""GPU parity of the chunked overlap-add demix (demix.hip) against the oracle.

Chunk inputs and the overlap-add are bit-exact with the oracle for identical chunk outputs
(both sum weight * output in double in chunk order and divide once). The driver
(stx_demix_track, RoFormer::separate) is checked with a per-stem-gain separator (bit-exact),
the identity separator under shifts, the complement stem, progress/cancel and error codes.
"""
import os

import numpy as np
import pytest

import oracle_lib
import stx
import synth
from hip_util import d2d
from metrics import snr_db

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def od():
    return oracle_lib.demix()


def dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


# The last two cover 8 chunks over 4 samples (the limit of the 4-sample kernel) and 11 (the
# kernel for any overlap).
# Chunks covering 4 consecutive samples, ceil((chunk + 3) / step): 5, 5, 2, 5, 3, 4, 5, 8, 11
# (the generic kernel), 6, 7, 2, and 1 with gaps between the chunks (step > chunk: uncovered
# samples are 0/0 -> 0).
CASES = [(7938000, 352800, 88200), (1000, 100, 25), (1000, 100, 100), (150, 100, 25), (60, 100, 50),
         (1001, 97, 31), (100000, 8000, 2000), (5003, 64, 9), (2000, 100, 10), (1000, 100, 20), (1000, 100, 17),
         (4000, 400, 400), (1000, 100, 152)]


@pytest.mark.parametrize("length,chunk,step", CASES)
def test_chunks_bit_exact(device, od, length, chunk, step):
    mix = synth.normal(length % 1000 + 3, (2, length), 0.3)
    plan = stx.Demix(length, 2, chunk, step)
    got = host(plan.chunks(dev(mix, device)))
    assert np.array_equal(got, od.chunks(mix, chunk, step))
    if plan.n_chunks > 3:                              # a sub-range
        got2 = host(plan.chunks(dev(mix, device), first=2, count=plan.n_chunks - 3))
        assert np.array_equal(got2, got[2:plan.n_chunks - 1])


@pytest.mark.parametrize("length,chunk,step", CASES)
def test_overlap_add_bit_exact(device, od, length, chunk, step):
    S = 4 if length > 1000000 else 3                   # the 180 s song: 4 stems, 1.08 GB of chunk outputs
    plan = stx.Demix(length, 2, chunk, step)
    y = synth.uniform(length % 977, (plan.n_chunks, S, 2, chunk))
    y[0, 0, 0, :3] = np.nan                             # non-finite outputs propagate like the reference
    got = host(plan.overlap_add(dev(y, device)))
    want = od.ola(y, length, chunk, step)
    assert np.array_equal(got, want, equal_nan=True)


def gains_separator(gains, C, chunk, batch, device):
    import torch
    g = torch.tensor(gains, dtype=torch.float32, device=device)[None, :, None, None]
    buf = torch.empty((batch, C, chunk), dtype=torch.float32, device=device)

    def sep(parts, first, count, y, stream):
        d2d(buf.data_ptr(), parts, count * C * chunk * 4, stream)
        yt = (g * buf[:count, None]).contiguous()
        d2d(y, yt.data_ptr(), yt.numel() * 4, stream)
        return 0
    return sep


@pytest.mark.parametrize("complement", [False, True])
def test_track_gains_bit_exact(device, od, complement):
    C, length, chunk = 2, 100003, 8000
    gains = [0.5, -1.25, 2.0]
    mix = synth.sines_plus_pink(9, C, length)
    out = host(stx.demix_track(dev(mix, device), chunk, 4, 3, gains_separator(gains, C, chunk, 5, device),
                               complement=complement, batch=5))
    step = stx.demix_step(chunk, 4)
    parts = od.chunks(mix, chunk, step)
    y = np.array(gains, np.float32)[None, :, None, None] * parts[:, None]
    want = od.ola(y, length, chunk, step)
    assert np.array_equal(out[:3], want)
    if complement:
        assert np.array_equal(out[3], mix - want[0])


def test_track_shifts_identity(device):
    C, length, chunk = 2, 30000, 4000
    mix = synth.normal(21, (C, length), 0.2)
    out = host(stx.demix_track(dev(mix, device), chunk, 2, 1, gains_separator([1.0], C, chunk, 3, device),
                               sample_rate=8000, batch=3, shifts=2, seed=5))
    assert np.max(np.abs(out[0] - mix)) <= 2e-7 * np.max(np.abs(mix))


def test_track_progress_and_cancel(device):
    C, length, chunk = 1, 20000, 2000
    mix = dev(synth.normal(22, (C, length), 0.2), device)
    seen = []
    step = stx.demix_step(chunk, 2)
    total = stx.demix_plan(length, chunk, step)[0]["n_chunks"]
    stx.demix_track(mix, chunk, 2, 1, gains_separator([1.0], C, chunk, 4, device), batch=4,
                    progress=lambda d, t: seen.append((d, t)))
    assert seen == [(d, total) for d in range(1, total)] + [(total, total)]
    calls = []

    def cancel():
        calls.append(1)
        return len(calls) >= 3
    with pytest.raises(stx.StxError) as e:
        stx.demix_track(mix, chunk, 2, 1, gains_separator([1.0], C, chunk, 4, device), batch=1,
                        should_cancel=cancel)
    assert e.value.status == stx.STATUS_CANCELLED and len(calls) == 3


def test_track_errors(device):
    import torch
    mix = torch.zeros((2, 0), dtype=torch.float32, device=device)
    with pytest.raises(stx.StxError) as e:
        stx.demix_track(mix, 1000, 2, 1, lambda *a: 0)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    mix = torch.zeros((2, 5000), dtype=torch.float32, device=device)
    with pytest.raises(stx.StxError) as e:
        stx.demix_track(mix, 1000, 2, 1, lambda *a: 0, overlap=1.0)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    with pytest.raises(stx.StxError) as e:
        stx.demix_track(mix, 1000, 2, 1, lambda *a: 7)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR


# The full-song workload: 180 s stereo (sum of 8 seeded sines + pink noise), 352,800-sample
# chunks at num_overlap 4 (step 88,200: 96 chunks), 4 stems (src/roformer.cpp:286-351,436-486).
SONG, CHUNK, SR = 7938000, 352800, 44100
NFFT, HOP = 2048, 441


def test_track_c5_gains_bit_exact(device, od):
    """stx_demix_track on the 180 s song with a 4-stem separator of seeded per-stem gains: the
    chunk table, the chunk inputs and the overlap-add are the oracle's bit for bit."""
    C = 2
    gains = [0.75, -0.5, 1.25, 0.3125]
    mix = synth.sines_plus_pink(5, C, SONG)
    out = host(stx.demix_track(dev(mix, device), CHUNK, 4, 4, gains_separator(gains, C, CHUNK, 8, device), batch=8))
    step = stx.demix_step(CHUNK, 4)
    assert step == 88200
    parts = od.chunks(mix, CHUNK, step)
    assert parts.shape[0] == 96
    y = np.array(gains, np.float32)[None, :, None, None] * parts[:, None]
    want = od.ola(y, SONG, CHUNK, step)
    assert np.array_equal(out, want)


def band_separator(masks, bands, C, chunk, batch, device):
    """The RoFormer spectral path as a 4-stem separator: per chunk, stx_torch_stft (2048/441),
    scatter-average + complex apply of fixed per-stem band masks, stx_torch_istft per stem."""
    import torch
    fft = stx.FFT(NFFT)
    S = masks.shape[1]
    F = NFFT // 2 + 1
    buf = torch.empty((batch, C, chunk), dtype=torch.float32, device=device)

    def sep(parts, first, count, y, stream):
        d2d(buf.data_ptr(), parts, count * C * chunk * 4, stream)
        for i in range(count):
            spec = stx.torch_stft(fft, buf[i], HOP, layout=stx.T_MAJOR)                  # [C][T][F]
            T = spec.shape[1]
            ys = bands.scatter_apply(masks, spec[None], T)[0]                            # [S][C][T][F]
            yy = stx.torch_istft(fft, ys.reshape(S * C, T, F), HOP, layout=stx.T_MAJOR)   # [S C][chunk]
            d2d(y + i * S * C * chunk * 4, yy.data_ptr(), S * C * chunk * 4, stream)
        return 0
    return sep


def test_track_c5_band_masks(device, od):
    """stx_demix_track on the 180 s song with the c3 spectral path as the separator: 4 stems of
    seeded band masks (uniform [-1, 1], 60 mel bands) applied to every chunk's STFT. Against
    the oracle composed the same way (double STFT, band scatter-average + apply, double iSTFT,
    then the overlap-add): per-stem SNR >= 110 dB."""
    from concurrent.futures import ThreadPoolExecutor
    C, S = 2, 4
    sizes, freqs = stx.mel_band_map(SR, NFFT, 60)
    bands = stx.Bands(sizes, freqs, NFFT // 2 + 1, C)
    T = CHUNK // HOP + 1
    masks_h = synth.uniform(77, (1, S, bands.total_feat * T))
    mix = synth.sines_plus_pink(6, C, SONG)
    out = host(stx.demix_track(dev(mix, device), CHUNK, 4, S,
                               band_separator(dev(masks_h, device), bands, C, CHUNK, 4, device), batch=4))
    step = stx.demix_step(CHUNK, 4)
    parts = od.chunks(mix, CHUNK, step)
    orc, ob = oracle_lib.oracle(), oracle_lib.bands()
    y = np.empty((parts.shape[0], S, C, CHUNK), dtype=np.float32)

    def chunk_ref(i):
        z = np.stack([orc.torch_stft(parts[i, c], NFFT, HOP) for c in range(C)])          # [C][F][T]
        ys = ob.scatter_apply(sizes, freqs, masks_h[0], z)                               # [S][C][F][T]
        for s in range(S):
            for c in range(C):
                y[i, s, c] = orc.torch_istft(ys[s, c], NFFT, HOP)
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        list(ex.map(chunk_ref, range(parts.shape[0])))
    want = od.ola(y, SONG, CHUNK, step)
    for s in range(S):
        assert snr_db(out[s], want[s]) >= 110.0, s
