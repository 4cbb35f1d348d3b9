"""CPU checks of the band path: pins the oracle (oracle/band_oracle.c) and compares the
library's host-side band maps and tables (stems.cpp_amd, stx_mel_band_map / stx_bs_band_map /
stx_bands_layout) with it bit for bit.

Mel map pins (librosa is not installed, so exact librosa-version behaviour stays unpinned):
the counts the survey of the reference restated on its own, an independent vectorised float32
restatement of librosa.filters.mel below, and the margin between bin frequencies and mel
vertices that makes the map insensitive to ulp-level log/exp differences.
"""
import numpy as np
import pytest

import oracle_lib
import stx
import synth

SR, NFFT, NMELS = 44100, 2048, 60
# BSRoformer's default freqs_per_bands (sums to 1025).
BS_FPB = [2] * 24 + [4] * 12 + [12] * 8 + [24] * 8 + [48] * 8 + [128, 129]


@pytest.fixture(scope="module")
def ob():
    return oracle_lib.bands()


def librosa_like_mel_mask(sr, n_fft, n_mels):
    """Vectorised restatement of librosa.filters.mel (Slaney, float32 weights) > 0."""
    f_sp, min_log_hz = 200.0 / 3, 1000.0
    min_log_mel, logstep = min_log_hz / f_sp, np.log(6.4) / 27.0

    def hz_to_mel(f):
        f = np.asarray(f, dtype=np.float64)
        return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-300) / min_log_hz) / logstep, f / f_sp)

    def mel_to_hz(m):
        return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), f_sp * m)

    fftfreqs = np.fft.rfftfreq(n=n_fft, d=1.0 / sr)
    mel_f = mel_to_hz(np.linspace(hz_to_mel(0.0), hz_to_mel(sr / 2.0), n_mels + 2))
    fdiff = np.diff(mel_f)
    ramps = np.subtract.outer(mel_f, fftfreqs)
    w = np.zeros((n_mels, fftfreqs.size), dtype=np.float32)
    for i in range(n_mels):
        w[i] = np.maximum(0, np.minimum(-ramps[i] / fdiff[i], ramps[i + 2] / fdiff[i + 1]))
    w *= (2.0 / (mel_f[2:] - mel_f[:-2]))[:, None]
    w[0][0] = 1.0
    w[-1, -1] = 1.0
    return w > 0, mel_f, fftfreqs


def test_mel_map_matches_survey_counts(ob):
    sizes, freqs = ob.mel_band_map(SR, NFFT, NMELS)
    assert sizes.size == 60 and freqs.size == 1979
    assert list(sizes[:3]) == [7, 6, 6] and list(sizes[-2:]) == [122, 130]
    assert sizes.min() == 6 and sizes.max() == 130
    _, _, bpf = ob.layout(sizes, freqs, NFFT // 2 + 1, 2)
    assert int((bpf == 1).sum()) == 71 and int((bpf == 2).sum()) == 954 and bpf.min() >= 1
    assert int(sizes.sum()) * 2 * 2 == 7916


@pytest.mark.parametrize("sr,n_fft,n_mels", [(44100, 2048, 60), (44100, 2048, 64), (44100, 4096, 60),
                                             (48000, 2048, 60), (44100, 1024, 32)])
def test_mel_map_matches_independent_restatement(ob, sr, n_fft, n_mels):
    mask, _, _ = librosa_like_mel_mask(sr, n_fft, n_mels)
    sizes, freqs = ob.mel_band_map(sr, n_fft, n_mels)
    assert list(sizes) == [int(r.sum()) for r in mask]
    assert list(freqs) == [int(k) for r in mask for k in np.nonzero(r)[0]]


def test_mel_map_margin():
    # Interior bins sit >= 0.098 Hz from every mel vertex (bin spacing 21.5 Hz), so no ulp-level
    # difference in the vertex frequencies can move a bin in or out of a band.
    _, mel_f, fftfreqs = librosa_like_mel_mask(SR, NFFT, NMELS)
    d = np.abs(np.subtract.outer(mel_f[1:-1], fftfreqs))
    assert d.min() >= 0.098


@pytest.mark.parametrize("sr,n_fft,n_mels", [(44100, 2048, 60), (44100, 4096, 60), (48000, 2048, 64)])
def test_library_mel_map_bit_exact(ob, sr, n_fft, n_mels):
    s1, f1 = ob.mel_band_map(sr, n_fft, n_mels)
    s2, f2 = stx.mel_band_map(sr, n_fft, n_mels)
    assert np.array_equal(s1, s2) and np.array_equal(f1, f2)


def test_bs_band_map():
    freqs = stx.bs_band_map(BS_FPB, NFFT)
    assert np.array_equal(freqs, np.arange(1025, dtype=np.int32))
    with pytest.raises(stx.StxError) as e:
        stx.bs_band_map(BS_FPB[:-1], NFFT)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR


@pytest.mark.parametrize("kind", ["mel", "bs"])
@pytest.mark.parametrize("channels", [1, 2])
def test_library_layout_bit_exact(ob, kind, channels):
    if kind == "mel":
        sizes, freqs = ob.mel_band_map(SR, NFFT, NMELS)
    else:
        sizes, freqs = np.array(BS_FPB, np.int32), np.arange(1025, dtype=np.int32)
    a = ob.layout(sizes, freqs, NFFT // 2 + 1, channels)
    b = stx.bands_layout(sizes, freqs, NFFT // 2 + 1, channels)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    assert a[1][-1] == int(sizes.sum()) * channels * 2
    assert int(a[2].sum()) == freqs.size


def test_layout_errors():
    sizes, freqs = np.array([2, 3], np.int32), np.array([0, 1, 1, 2, 3], np.int32)
    with pytest.raises(stx.StxError) as e:          # sizes sum 5 != 4 freqs
        stx.bands_layout(sizes, freqs[:4], 8, 2)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR
    with pytest.raises(stx.StxError) as e:          # bin 3 out of range for 3 bins
        stx.bands_layout(sizes, freqs, 3, 2)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR


def random_table(seed, n_bins, n_bands):
    """Overlapping contiguous bands plus one band with repeated and unordered bins."""
    u = synth.uniform01(seed, 2 * n_bands)
    sizes, freqs = [], []
    for b in range(n_bands):
        start = int(u[2 * b] * (n_bins - 2))
        size = 1 + int(u[2 * b + 1] * min(6, n_bins - start - 1))
        sizes.append(size)
        freqs += list(range(start, start + size))
    sizes.append(4)
    freqs += [n_bins - 1, 0, 3, 3]
    return np.array(sizes, np.int32), np.array(freqs, np.int32)


def numpy_gather(sizes, freqs, z):
    C, F, T = z.shape
    out = []
    off = 0
    for s in sizes:
        fl = freqs[off:off + s]
        blk = z[:, fl, :]                                  # [C][s][T]
        blk = np.transpose(blk, (2, 1, 0))                 # [T][s][C]
        out.append(np.stack([blk.real, blk.imag], -1).astype(np.float32).reshape(-1))
        off += s
    return np.concatenate(out)


def numpy_scatter(sizes, freqs, masks, z, zero_dc):
    C, F, T = z.shape
    S = masks.shape[0]
    out = np.zeros((S, C, F, T), np.complex128)
    bpf = np.bincount(freqs, minlength=F)
    for st in range(S):
        acc = np.zeros((C, F, T), np.complex128)
        off = eoff = 0
        for s in sizes:
            din = s * C * 2
            m = masks[st, eoff * T:(eoff + din) * T].reshape(T, s, C, 2).astype(np.float64)
            for j in range(s):
                acc[:, freqs[off + j], :] += (m[:, j, :, 0] + 1j * m[:, j, :, 1]).T
            off += s
            eoff += din
        out[st] = z * (acc / np.maximum(bpf, 1)[None, :, None])
        if zero_dc:
            out[st, :, 0, :] = 0
    return out


@pytest.mark.parametrize("seed", [1, 2])
def test_oracle_gather_scatter_brute_force(ob, seed):
    sizes, freqs = random_table(seed, 17, 6)
    C, F, T, S = 2, 17, 5, 3
    v = synth.normal(seed, (2, C, F, T), 1.0).astype(np.float64)
    z = v[0] + 1j * v[1]
    feat = ob.gather(sizes, freqs, z)
    assert np.array_equal(feat, numpy_gather(sizes, freqs, z))
    masks = synth.uniform(seed + 10, (S, int(sizes.sum()) * C * 2 * T))
    for zd in (False, True):
        got = ob.scatter_apply(sizes, freqs, masks, z, zd)
        assert np.max(np.abs(got - numpy_scatter(sizes, freqs, masks, z, zd))) < 1e-12


def test_oracle_scatter_of_bin_constant_masks(ob):
    # Masks that repeat one value per (channel, bin, frame) in every band covering the bin
    # average back to that value exactly: out = z * v.
    sizes, freqs = ob.mel_band_map(SR, 256, 12)
    C, F, T = 2, 129, 4
    v = synth.uniform(3, (2, C, F, T)).astype(np.float64)
    val = v[0] + 1j * v[1]
    w = synth.normal(4, (2, C, F, T), 1.0).astype(np.float64)
    z = w[0] + 1j * w[1]
    masks = ob.gather(sizes, freqs, val)[None, :]
    got = ob.scatter_apply(sizes, freqs, masks, z)[0]
    assert np.array_equal(got, z * val.astype(np.complex64).astype(np.complex128))
