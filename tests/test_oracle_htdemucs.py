"""CPU checks that pin the HTDemucs pre/post-processing and split oracle
(oracle/htdemucs_oracle.c).

No reference test or golden vector covers HTDemucs::run's normalisation or separate()'s split
(the reference's own parity fixtures need the model). The oracle is pinned instead by:
torch.std's unbiased estimator for std_of; numpy float32 restatements of the normalise
formulas and of the weighted overlap-add (bit for bit: numpy's float32 operations round like
the reference's float ones); the triangular weights' closed form; the identity model, for which
split() must return the view it was given; and the TensorChunk rule the reference documents
(src/htdemucs.cpp:530-533), that the last segment is centre-padded with the audio before it.
"""
import numpy as np
import pytest

import oracle_lib
import synth

SEG = 343980          # 39/5 s at 44.1 kHz (src/htdemucs.cpp:313,317)


@pytest.fixture(scope="module")
def htd():
    return oracle_lib.htdemucs()


def test_mean_std_is_torch_unbiased(htd):
    import torch
    x = synth.normal(3, (2, 5000), 0.3) + 0.01
    m, s = htd.mean_std(x)
    t = torch.from_numpy(x.astype(np.float64))
    assert abs(m - t.mean().item()) <= 1e-15 * abs(m) + 1e-18
    assert abs(s - t.std(unbiased=True).item()) <= 1e-13 * s


def test_normalize_formulas_vs_numpy(htd):
    x = synth.normal(4, (3, 777), 2.0)
    m, s = htd.mean_std(x)
    want = ((x.astype(np.float64) - m) / (1e-5 + s)).astype(np.float32)
    assert np.array_equal(htd.normalize(x, m, s), want)
    spec = (synth.normal(5, (2, 16, 9), 1.0) + 1j * synth.normal(6, (2, 16, 9), 1.0)).astype(np.complex64)
    mag_raw = htd.cac_pack(spec)
    m2, s2 = htd.mean_std(mag_raw)
    want2 = ((mag_raw.astype(np.float64) - m2) / (1e-5 + s2)).astype(np.float32)
    assert np.array_equal(htd.cac_normalize(spec, m2, s2), want2)
    assert np.array_equal(want2[0], ((spec[0].real.astype(np.float64) - m2) / (1e-5 + s2)).astype(np.float32))
    assert np.array_equal(want2[3], ((spec[1].imag.astype(np.float64) - m2) / (1e-5 + s2)).astype(np.float32))


def test_denormalize_inverts_normalize(htd):
    spec = (synth.normal(7, (2, 8, 5), 1.0) + 1j * synth.normal(8, (2, 8, 5), 1.0)).astype(np.complex64)
    m, s = htd.mean_std(htd.cac_pack(spec))
    mag = htd.cac_normalize(spec, m, s)
    back = htd.cac_denormalize(mag[None], m, s)[0]
    # (v - m) / (1e-5 + s) * s + m differs from v by the 1e-5 and two roundings.
    assert np.max(np.abs(back - spec)) <= 1e-4 * np.max(np.abs(spec))
    ox = synth.normal(9, (3, 4, 8, 5), 1.0)
    got = htd.cac_denormalize(ox, 0.25, 1.5)
    assert np.array_equal(got[2, 1].real, (ox[2, 2].astype(np.float64) * 1.5 + 0.25).astype(np.float32))
    assert np.array_equal(got[2, 1].imag, (ox[2, 3].astype(np.float64) * 1.5 + 0.25).astype(np.float32))


def test_time_add(htd):
    t, y = synth.normal(10, (999,), 1.0), synth.normal(11, (999,), 1.0)
    got = htd.time_add(t, y, -0.1, 3.0)
    assert np.array_equal(got, (t.astype(np.float64) * 3.0 - 0.1).astype(np.float32) + y)


def test_mix_normalize(htd):
    import torch
    mix = synth.normal(12, (2, 4001), 0.2) + 0.05
    out, stats = htd.mix_normalize(mix)
    mono = (mix.astype(np.float64).sum(0) / 2).astype(np.float32)
    t = torch.from_numpy(mono.astype(np.float64))
    assert abs(stats[0] - t.mean().item()) <= 1e-14
    assert abs(stats[1] - t.std().item()) <= 1e-13 * stats[1]
    assert np.array_equal(out, ((mix.astype(np.float64) - stats[0]) / stats[1]).astype(np.float32))
    # Silence: std 0 -> floored at 1e-8.
    _, st0 = htd.mix_normalize(np.zeros((2, 10), np.float32))
    assert st0[0] == 0.0 and st0[1] == 1e-8


@pytest.mark.parametrize("seg", [SEG, 7, 8])
def test_split_weights_closed_form(htd, seg):
    w = htd.split_weights(seg)
    assert w.max() == 1.0
    assert np.array_equal(w, w[::-1]) or seg % 2 == 1 and np.array_equal(w[:-1], w[:-1][::-1])
    half = seg // 2
    raw = np.array([i + 1 if i < half else seg - i for i in range(seg)], np.float32)
    assert np.array_equal(w, raw / np.float32(raw.max()))


def test_split_count(htd):
    assert htd.split_count(7938000, SEG, 0.25) == (257985, 31)
    assert htd.split_count(100, 40, -1.0) == (30, 4)        # negative overlap means 0.25
    assert htd.split_count(100, 40, 1.0)[1] == -1


def np_segments(buf, offset, length, seg, stride):
    C, total = buf.shape
    out = []
    for off in range(0, length, stride):
        clen = min(seg, length - off)
        start = offset + off - (seg - clen) // 2
        j = np.arange(seg) + start
        ok = (j >= 0) & (j < total)
        part = np.zeros((C, seg), np.float32)
        part[:, ok] = buf[:, j[ok]]
        out.append(part)
    return np.stack(out)


def np_split_ola(y, length, seg, stride, w):
    n, tracks, _ = y.shape
    out = np.zeros((tracks, length), np.float32)
    sw = np.zeros(length, np.float32)
    for k, off in enumerate(range(0, length, stride)):
        clen = min(seg, length - off)
        trim = (seg - clen) // 2
        out[:, off:off + clen] += w[:clen] * y[k, :, trim:trim + clen]
        sw[off:off + clen] += w[:clen]
    return out / sw


@pytest.mark.parametrize("length,seg,stride,offset,total", [(1000, 300, 225, 0, 1000), (1000, 300, 225, 37, 1100),
                                                            (50, 300, 225, 0, 50), (901, 64, 48, 10, 950)])
def test_segments_and_ola_vs_numpy(htd, length, seg, stride, offset, total):
    buf = synth.normal(13, (2, total), 1.0)
    parts = htd.segments(buf, offset, length, seg, stride)
    assert np.array_equal(parts, np_segments(buf, offset, length, seg, stride))
    y = synth.normal(14, (parts.shape[0], 3, seg), 1.0)
    w = htd.split_weights(seg)
    assert np.array_equal(htd.split_ola(y, length, stride), np_split_ola(y, length, seg, stride, w))


def test_last_segment_padded_with_audio_before_it(htd):
    """TensorChunk.padded: the short last chunk is centred with real samples on both sides."""
    length, seg, stride = 1000, 300, 225
    buf = np.arange(1, 1 + 2 * length, dtype=np.float32).reshape(2, length)
    parts = htd.segments(buf, 0, length, seg, stride)
    off = 4 * stride                                   # last chunk: 100 samples
    clen = length - off
    start = off - (seg - clen) // 2
    assert parts[-1, 0, 0] == buf[0, start] != 0.0     # audio from before the chunk, not silence
    assert np.all(parts[-1, :, (seg - clen) // 2 + clen:] == 0.0)  # beyond the buffer: zeros


def test_identity_model_returns_view(htd):
    """split() of a model that returns its input gives back the view (to a float rounding)."""
    length, seg, stride = 2000, 512, 384
    buf = synth.normal(15, (2, length), 1.0)
    parts = htd.segments(buf, 0, length, seg, stride)
    y = np.concatenate([parts, parts], axis=1)         # two "sources", [n][S*C][seg]
    out = htd.split_ola(y, length, stride)
    assert np.max(np.abs(out[:2] - buf)) <= 4e-7 * np.max(np.abs(buf))
    assert np.array_equal(out[:2], out[2:])


def test_shift_offsets_range_and_determinism(htd):
    a = htd.shift_offsets(7, 22050, 2, 5)
    b = htd.shift_offsets(7, 22050, 2, 5)
    assert np.array_equal(a, b) and a.min() >= 0 and a.max() <= 22050
    # One generator across models: model 1 continues the sequence of model 0.
    c = htd.shift_offsets(7, 22050, 1, 10)
    assert np.array_equal(a.reshape(-1), c.reshape(-1))


def test_separate_identity_bag(htd):
    """Two models that both return the input for every source, any weights: separate() gives the
    mix back (normalise, split, shifts, bag and denormalise undo each other to float rounding)."""
    mix = synth.normal(16, (2, 3000), 0.3) + 0.01
    bag = np.array([[1.0, 0.5], [0.25, 2.0]], np.float32)
    ident = lambda m, parts: np.concatenate([parts, parts], axis=1)
    out = htd.separate(mix, 512, bag, ident, sample_rate=400, shifts=2, seed=3)
    for s in range(2):
        assert np.max(np.abs(out[s] - mix)) <= 2e-6 * np.max(np.abs(mix))
