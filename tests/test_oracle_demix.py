"""CPU checks of the chunked overlap-add demix: pins the oracle (oracle/demix_oracle.c) and
compares the library's host-side chunk table and fade window (stx_demix_plan /
stx_demix_window) with it bit for bit.

Pins: the chunk table the survey of the reference derived for the 180 s config, torch's own
float32 linspace for the fade (the reference computes it "the way torch does",
src/roformer.cpp:303), an independent numpy restatement of the loop on small sizes, and the
identity separator (the overlap-add of unchanged chunks returns the input).
"""
import numpy as np
import pytest

import oracle_lib
import stx
import synth


@pytest.fixture(scope="module")
def od():
    return oracle_lib.demix()


def test_chunk_table_full_song_config():
    # 180 s stereo at 44.1 kHz, chunk 352,800, num_overlap 4.
    step = stx.demix_step(352800, 4)
    assert step == 88200
    g, t = stx.demix_plan(7938000, 352800, step)
    assert g["border"] == 264600 and g["fade"] == 35280 and g["reflect_border"] == 1
    assert g["padded_len"] == 8467200 and g["n_chunks"] == 96
    assert np.array_equal(t["start"], np.arange(96) * 88200)
    no_fade_out = t["start"][t["fade_out"] == 0]
    assert list(no_fade_out) == [8114400, 8202600, 8290800, 8379000]
    assert t["fade_in"][0] == 0 and t["fade_in"][1:].all()
    short = [(int(c["length"]), int(c["pad_mode"])) for c in t if c["length"] < 352800]
    assert short == [(264600, stx.CHUNK_REFLECT), (176400, stx.CHUNK_ZERO), (88200, stx.CHUNK_ZERO)]


@pytest.mark.parametrize("length,chunk,step", [(7938000, 352800, 88200), (1000, 100, 25), (1000, 100, 100),
                                               (150, 100, 25), (60, 100, 50), (1001, 97, 31)])
def test_plan_against_oracle_and_closed_form(od, length, chunk, step):
    g, t = stx.demix_plan(length, chunk, step)
    assert g["n_chunks"] == od.n_chunks(length, chunk, step)
    border = chunk - step
    pad = length > 2 * border and border > 0
    Lp = length + 2 * border if pad else length
    assert g["padded_len"] == Lp and g["n_chunks"] == -(-Lp // step)
    for k, c in enumerate(t):
        i = k * step
        assert c["start"] == i and c["length"] == min(chunk, Lp - i)
        mode = stx.CHUNK_FULL if c["length"] == chunk else (
            stx.CHUNK_REFLECT if c["length"] > chunk // 2 + 1 else stx.CHUNK_ZERO)
        assert c["pad_mode"] == mode
        assert c["fade_out"] == (0 if (i != 0 and i + chunk >= Lp) else 1)


@pytest.mark.parametrize("chunk", [352800, 100, 15, 10, 9, 1001])
def test_window_bit_exact_and_torch_linspace(od, chunk):
    import torch
    w = stx.demix_window(chunk)
    assert np.array_equal(w, od.window(chunk))
    fade = chunk // 10
    if fade > 1:
        # The first half, i * step, is one rounding in both. For the second half the reference
        # rounds twice (1 - round(k * step), no FMA) while torch's CPU kernel fuses it into one
        # rounding, so the two may differ by one ulp there; the reference's own value is the
        # contract and the library matches it bit for bit above.
        lin = torch.linspace(0, 1, fade, dtype=torch.float32).numpy()
        h = fade // 2
        assert np.array_equal(w[:h], lin[:h])
        ulp = np.abs(w[:fade].view(np.int32).astype(np.int64) - lin.view(np.int32).astype(np.int64))
        assert ulp.max() <= 1
        assert np.array_equal(w[chunk - fade:], w[:fade][::-1])
    elif fade == 1:
        assert w[0] == 0.0 and w[-1] == 0.0        # fade_in stays zero-initialised
    assert np.all(w[fade:chunk - fade] == 1.0)


def test_step_rule():
    assert stx.demix_step(352800, 2) == 176400
    assert stx.demix_step(352800, 4, -1.0) == 88200
    assert stx.demix_step(352800, 4, 0.5) == 176400
    assert stx.demix_step(1000, 4, 0.3333) == 667
    assert stx.demix_step(10, 4, 0.99) == 1
    assert stx.demix_step(352800, 4, 1.0) == 0


def numpy_demix(mix, chunk, step, sep):
    """Independent restatement of src/roformer.cpp:286-351 with a separator function."""
    C, length = mix.shape
    fade, border = chunk // 10, chunk - step
    pad = length > 2 * border and border > 0
    x = np.pad(mix.astype(np.float64), ((0, 0), (border, border)), mode="reflect").astype(np.float32) if pad else mix
    Lp = x.shape[1]
    fade_in = np.zeros(fade, np.float32)
    if fade > 1:
        stp = np.float32(1.0) / np.float32(fade - 1)
        for i in range(fade):
            fade_in[i] = np.float32(i) * stp if i < fade // 2 else np.float32(1.0) - np.float32(fade - 1 - i) * stp
    window = np.ones(chunk, np.float32)
    for i in range(fade):
        window[i] *= fade_in[i]
        window[chunk - 1 - i] *= fade_in[i]
    result, counter = None, np.zeros(Lp)
    for i in range(0, Lp, step):
        length_i = min(chunk, Lp - i)
        part = np.zeros((C, chunk), np.float32)
        part[:, :length_i] = x[:, i:i + length_i]
        if length_i < chunk and length_i > chunk // 2 + 1:
            part = np.pad(x[:, i:i + length_i].astype(np.float64), ((0, 0), (0, chunk - length_i)),
                          mode="reflect").astype(np.float32)
        y = sep(part)
        if result is None:
            result = np.zeros((y.shape[0], C, Lp))
        w = window.copy()
        if i == 0:
            w[:fade] = 1
        elif i + chunk >= Lp:
            w[chunk - fade:] = 1
        result[:, :, i:i + length_i] += y[:, :, :length_i].astype(np.float64) * w[:length_i]
        counter[i:i + length_i] += w[:length_i]
    off = border if pad else 0
    with np.errstate(invalid="ignore", divide="ignore"):
        v = result[:, :, off:off + length] / counter[off:off + length]
    return np.nan_to_num(v, nan=0.0, posinf=0.0, neginf=0.0).astype(np.float32)


@pytest.mark.parametrize("length,chunk,step", [(1000, 100, 25), (1000, 100, 100), (150, 100, 25),
                                               (60, 100, 50), (1001, 97, 31)])
def test_oracle_against_numpy_restatement(od, length, chunk, step):
    mix = synth.normal(length + chunk, (2, length), 0.3)
    gains = np.array([0.5, -1.25, 2.0], np.float32)
    parts = od.chunks(mix, chunk, step)
    y = gains[None, :, None, None] * parts[:, None, :, :]
    got = od.ola(y, length, chunk, step)
    want = numpy_demix(mix, chunk, step, lambda p: gains[:, None, None] * p[None])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("length,chunk,step", [(1000, 100, 25), (20000, 1000, 250), (1001, 97, 31)])
def test_identity_separator_returns_input(od, length, chunk, step):
    mix = synth.normal(7, (2, length), 0.3)
    out = od.ola(od.chunks(mix, chunk, step)[:, None], length, chunk, step)[0]
    assert np.max(np.abs(out - mix)) <= 1e-7 * np.max(np.abs(mix))
