"""GPU parity of the HTDemucs pre/post-processing and split (htdemucs.hip) against the oracle.

Bars: the device statistics (mean, unbiased std) within 1e-12 relative of the oracle's
sequential double sums (only the summation order differs); every normalised, denormalised or
added value bit-exact against the oracle given the same statistics, and within rel_err 1e-6
with the oracle's own; segments and the split overlap-add bit-exact.

Shapes: one c1 segment (stereo, 343,980 samples, n_fft 4096: spectrum [2][2048][336], four
sources) and the 180 s stereo song split into 31 segments of 343,980 samples at overlap 0.25
(stride 257,985), with and without a shift view.
"""
import numpy as np
import pytest

import oracle_lib
import stx
import synth
from metrics import rel_err

pytestmark = pytest.mark.gpu

SEG, NFFT = 343980, 4096
SONG = 7938000


@pytest.fixture(scope="module")
def htd():
    return oracle_lib.htdemucs()


def dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def close_stats(got, want):
    return abs(got[0] - want[0]) <= 1e-12 * max(abs(want[0]), want[1]) and abs(got[1] - want[1]) <= 1e-12 * want[1]


def test_cac_normalize_c1(device, htd):
    """src/htdemucs.cpp:424-436 on the device spectrum of one c1 segment."""
    x = dev(synth.normal(1, (2, SEG), 0.1), device)
    fft = stx.FFT(NFFT)
    spec = stx.htdemucs_spec(fft, x)                                   # complex64 [2, 2048, 336]
    mag, stats = stx.htdemucs_cac_normalize(spec)
    sh = host(spec)
    st = host(stats)
    want_stats = htd.mean_std(htd.cac_pack(sh))
    assert close_stats(st, want_stats)
    assert np.array_equal(host(mag), htd.cac_normalize(sh, st[0], st[1]))
    assert rel_err(host(mag), htd.cac_normalize(sh, *want_stats)) <= 1e-6


@pytest.mark.parametrize("C,F,T", [(2, 33, 77), (2, 64, 51), (3, 2049, 5), (1, 7, 3)])
def test_cac_normalize_ragged(device, htd, C, F, T):
    """Spectra whose float count is not a multiple of a block's chunk, with an odd bins x frames
    product (each float placed on its own) and an even one (re/im pairs)."""
    import torch
    z = synth.normal(C * F + T, (C, F, T, 2), 1.0) * 3 + 0.5
    sh = (z[..., 0] + 1j * z[..., 1]).astype(np.complex64)
    mag, stats = stx.htdemucs_cac_normalize(torch.from_numpy(sh).to(device))
    st = host(stats)
    assert close_stats(st, htd.mean_std(htd.cac_pack(sh)))
    assert np.array_equal(host(mag), htd.cac_normalize(sh, st[0], st[1]))


def test_wave_normalize_c1(device, htd):
    xh = synth.normal(2, (2, SEG), 0.1) + 0.003
    y, stats = stx.htdemucs_wave_normalize(dev(xh, device))
    st = host(stats)
    assert close_stats(st, htd.mean_std(xh))
    assert np.array_equal(host(y), htd.normalize(xh, st[0], st[1]))


@pytest.mark.parametrize("n", [2, 3, 8191, 8192, 8193, 100003, 5000001])   # last: too large for one pass
def test_wave_normalize_ragged(device, htd, n):
    xh = synth.normal(3, (n,), 1.0) * 5 + 2
    y, stats = stx.htdemucs_wave_normalize(dev(xh, device))
    st = host(stats)
    assert close_stats(st, htd.mean_std(xh))
    assert np.array_equal(host(y), htd.normalize(xh, st[0], st[1]))


def test_normalize_without_grid_sync(device, htd, monkeypatch):
    """STX_NO_GRID_SYNC=1 sends one segment's normalisations to the two-kernel path."""
    monkeypatch.setenv("STX_NO_GRID_SYNC", "1")
    xh = synth.normal(9, (2, SEG), 0.1) - 0.02
    y, stats = stx.htdemucs_wave_normalize(dev(xh, device))
    st = host(stats)
    assert close_stats(st, htd.mean_std(xh))
    assert np.array_equal(host(y), htd.normalize(xh, st[0], st[1]))
    x = dev(synth.normal(10, (2, SEG), 0.1), device)
    spec = stx.htdemucs_spec(stx.FFT(NFFT), x)
    mag, stats = stx.htdemucs_cac_normalize(spec)
    sh, st = host(spec), host(stats)
    assert close_stats(st, htd.mean_std(htd.cac_pack(sh)))
    assert np.array_equal(host(mag), htd.cac_normalize(sh, st[0], st[1]))


def test_normalize_forced_fallback(device, htd, monkeypatch):
    """STX_GRID_SYNC_SPIN_LIMIT=0 makes the single-pass blocks give up their waits at the first
    look; each then computes the totals from the input itself, in the same order: the same bits
    as the normal run, and the workspace counts the fallbacks."""
    xh = synth.normal(11, (2, SEG), 0.1) + 0.01
    x = dev(xh, device)
    y1, st1 = stx.htdemucs_wave_normalize(x)
    spec = stx.htdemucs_spec(stx.FFT(NFFT), dev(synth.normal(12, (2, SEG), 0.1), device))
    m1, sc1 = stx.htdemucs_cac_normalize(spec)
    ws = stx.workspace(stx.lib().stx_htdemucs_norm_workspace_size(2 * 2 * 2048 * 336), device)
    monkeypatch.setenv("STX_GRID_SYNC_SPIN_LIMIT", "0")
    y2, st2 = stx.htdemucs_wave_normalize(x, workspace=ws)
    m2, sc2 = stx.htdemucs_cac_normalize(spec, workspace=ws)
    monkeypatch.delenv("STX_GRID_SYNC_SPIN_LIMIT")
    assert stx.grid_sync_fallbacks(ws) > 0
    assert np.array_equal(host(y1), host(y2)) and np.array_equal(host(st1), host(st2))
    assert np.array_equal(host(m1), host(m2)) and np.array_equal(host(sc1), host(sc2))
    assert close_stats(host(st1), htd.mean_std(xh))


def test_normalize_in_place(device, htd):
    """Output over its input: the two-kernel path (a single-pass block may re-read x)."""
    xh = synth.normal(13, (2, SEG), 0.1) - 0.005
    x = dev(xh, device)
    y, stats = stx.htdemucs_wave_normalize(x, out=x)
    st = host(stats)
    assert close_stats(st, htd.mean_std(xh))
    assert np.array_equal(host(y), htd.normalize(xh, st[0], st[1]))


def test_normalize_in_place_many_waves(device, htd):
    """In-place calls large enough that the normalising blocks run in several waves (2 x 180 s
    stereo waveforms: 3,876 blocks; the 180 s stereo mix: 1,938 blocks of 8,192 values, 32 per
    thread): output and statistics bit-equal to the out-of-place call, whose blocks never see
    their own output. A late block must not take an already-normalised x[0] as its shift."""
    import torch
    xh = synth.normal(14, (2, 2 * SONG), 0.1) + 0.02
    x = dev(xh, device)
    y_ref, st_ref = stx.htdemucs_wave_normalize(x)
    y, st = stx.htdemucs_wave_normalize(x, out=x)
    assert y.data_ptr() == x.data_ptr()
    assert np.array_equal(host(st), host(st_ref)) and np.array_equal(host(y), host(y_ref))
    assert close_stats(host(st), htd.mean_std(xh))
    del x, y, y_ref
    mix = synth.sines_plus_pink(5, 2, SONG)
    m = dev(mix, device)
    o_ref, s_ref = stx.htdemucs_mix_normalize(m)
    o, s = stx.htdemucs_mix_normalize(m, out=m)
    assert np.array_equal(host(s), host(s_ref)) and np.array_equal(host(o), host(o_ref))
    torch.cuda.synchronize()


def test_normalize_overlap_refused(device):
    """An output that overlaps its input without being the same buffer is refused (blocks would
    overwrite values other blocks have yet to read), and so is any overlap for the CaC pack,
    whose planes move every value."""
    import torch
    x = torch.zeros(2 * 100000, dtype=torch.float32, device=device)
    with pytest.raises(stx.StxError) as e:
        stx.htdemucs_wave_normalize(x[:100000], out=x[1:100001])
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT and "overlaps" in e.value.message
    spec = torch.zeros((2, 64, 100), dtype=torch.complex64, device=device)
    with pytest.raises(stx.StxError) as e:
        stx.htdemucs_cac_normalize(spec, out=torch.view_as_real(spec).reshape(4, 64, 100))
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT and "overlaps" in e.value.message


def test_mix_normalize_song(device, htd):
    """src/htdemucs.cpp:539-549 on the 180 s stereo song."""
    mix = synth.sines_plus_pink(5, 2, SONG)
    out, stats = stx.htdemucs_mix_normalize(dev(mix, device))
    want, wstats = htd.mix_normalize(mix)
    st = host(stats)
    assert close_stats(st, wstats)
    assert rel_err(host(out), want) <= 1e-6


@pytest.mark.parametrize("C", [1, 2])
def test_mix_normalize_single_pass_same_bits(device, htd, C, monkeypatch):
    """The single-pass mix normalise (one and two channels, a tail chunk of 1,000,003 % 8,192
    samples) gives the two-kernel path's bits, and so does its fallback when every wait gives
    up at the first look (STX_GRID_SYNC_SPIN_LIMIT=0: each block then forms all chunk sums
    itself, in the same order); the workspace counts the fallbacks."""
    n = 1_000_003
    mix = synth.sines_plus_pink(20 + C, C, n)
    m = dev(mix, device)
    o1, s1 = stx.htdemucs_mix_normalize(m)
    monkeypatch.setenv("STX_NO_GRID_SYNC", "1")
    o2, s2 = stx.htdemucs_mix_normalize(m)
    monkeypatch.delenv("STX_NO_GRID_SYNC")
    ws = stx.workspace(stx.lib().stx_htdemucs_norm_workspace_size(n), device)
    monkeypatch.setenv("STX_GRID_SYNC_SPIN_LIMIT", "0")
    o3, s3 = stx.htdemucs_mix_normalize(m, workspace=ws)
    monkeypatch.delenv("STX_GRID_SYNC_SPIN_LIMIT")
    assert stx.grid_sync_fallbacks(ws) > 0
    for o, s in ((o2, s2), (o3, s3)):
        assert np.array_equal(host(o), host(o1)) and np.array_equal(host(s), host(s1))
    want, wstats = htd.mix_normalize(mix)
    assert close_stats(host(s1), wstats)
    assert rel_err(host(o1), want) <= 1e-6


def test_mix_normalize_silence_and_errors(device):
    import torch
    out, stats = stx.htdemucs_mix_normalize(torch.zeros((2, 1000), device=device))
    st = host(stats)
    assert st[0] == 0.0 and st[1] == 1e-8
    assert np.all(host(out) == 0.0)
    with pytest.raises(stx.StxError) as e:
        stx.htdemucs_mix_normalize(torch.zeros((2, 0), device=device))
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT and "empty input" in e.value.message


def test_denormalize_and_time_add_c1(device, htd):
    """src/htdemucs.cpp:465-470 for four sources: denormalise, iSTFT, time branch + add."""
    import torch
    S, C, F, T = 4, 2, 2048, 336
    ox = dev(synth.normal(4, (S, 2 * C, F, T), 1.0), device)
    stats = torch.tensor([0.0123, 0.456], dtype=torch.float64, device=device)
    spec = stx.htdemucs_cac_denormalize(ox, stats)
    want = htd.cac_denormalize(host(ox), 0.0123, 0.456)
    assert np.array_equal(host(spec), want)
    fft = stx.FFT(NFFT)
    y = stx.htdemucs_ispec(fft, spec.reshape(S * C, F, T), SEG)
    xt = dev(synth.normal(5, (S * C, SEG), 1.0), device)
    tstats = torch.tensor([-0.002, 0.09], dtype=torch.float64, device=device)
    out = stx.htdemucs_time_add(xt, y, tstats)
    assert np.array_equal(host(out), htd.time_add(host(xt), host(y), -0.002, 0.09))


@pytest.mark.parametrize("shifted", [False, True])
def test_segments_song(device, htd, shifted):
    """TensorChunk views of the 180 s song: the plain split and one shift view (the mix padded
    by sr/2 on both sides, src/htdemucs.cpp:613-621)."""
    mix = synth.sines_plus_pink(6, 2, SONG)
    if shifted:
        max_shift, off = 22050, 12345
        buf = np.zeros((2, SONG + 2 * max_shift), np.float32)
        buf[:, max_shift:max_shift + SONG] = mix
        offset, length = off, SONG + max_shift - off
    else:
        buf, offset, length = mix, 0, SONG
    stride, n = stx.htdemucs_split_plan(length, SEG, 0.25)
    assert (stride, n) == htd.split_count(length, SEG, 0.25)
    bd = dev(buf, device)
    want = htd.segments(buf, offset, length, SEG, stride)
    got = host(stx.htdemucs_segments(bd, offset, length, SEG, stride))
    assert np.array_equal(got, want)
    part = host(stx.htdemucs_segments(bd, offset, length, SEG, stride, first=n - 2, count=2))
    assert np.array_equal(part, want[n - 2:])


@pytest.mark.parametrize("length,tracks", [(SONG, 8), (SEG, 8), (1000, 3), (SEG + 1, 2)])
def test_split_overlap_add(device, htd, length, tracks):
    """src/htdemucs.cpp:594-606, bit-exact: float products and sums in chunk order."""
    seg = SEG if length >= SEG else 300
    stride, n = stx.htdemucs_split_plan(length, seg, 0.25)
    y = synth.normal(7, (n, tracks, seg), 1.0)
    got = host(stx.htdemucs_split_overlap_add(dev(y, device), length, stride))
    assert np.array_equal(got, htd.split_ola(y, length, stride))


def test_split_identity_model(device):
    """A model that returns its input: split() gives the normalised mix back."""
    import torch
    mix = dev(synth.sines_plus_pink(8, 2, 1_000_000), device)
    norm, stats = stx.htdemucs_mix_normalize(mix)
    stride, n = stx.htdemucs_split_plan(1_000_000, SEG, 0.25)
    parts = stx.htdemucs_segments(norm, 0, 1_000_000, SEG, stride)
    y = torch.cat([parts, parts], dim=1).contiguous()                   # two sources
    out = host(stx.htdemucs_split_overlap_add(y, 1_000_000, stride))
    nh = host(norm)
    assert np.max(np.abs(out[:2] - nh)) <= 4e-7 * np.max(np.abs(nh))


def test_split_errors(device):
    with pytest.raises(stx.StxError) as e:
        stx.htdemucs_split_plan(1000, 300, 1.0)
    assert "overlap must be < 1" in e.value.message


# --------------------------------------------------------------------- separate() driver
def gain_model(gains, C, seg, batch, device):
    """Model m returns gains[m][s] * segment for source s: linear, so the oracle composes it."""
    import torch
    from hip_util import d2d
    g = torch.tensor(gains, dtype=torch.float32, device=device)        # [n_models][S]
    buf = torch.empty((batch, C, seg), dtype=torch.float32, device=device)

    def forward(model, parts, count, y, stream):
        d2d(buf.data_ptr(), parts, count * C * seg * 4, stream)
        yt = (g[model][None, :, None, None] * buf[:count, None]).contiguous()   # [count][S][C][seg]
        d2d(y, yt.data_ptr(), yt.numel() * 4, stream)
        return 0

    def np_model(m, parts):
        gm = np.array(gains, np.float32)[m]
        y = gm[None, :, None, None] * parts[:, None]
        return y.reshape(parts.shape[0], -1, parts.shape[2])
    return forward, np_model


@pytest.mark.parametrize("shifts,n_models", [(0, 1), (2, 2)])
def test_separate_gain_models_vs_oracle(device, htd, shifts, n_models):
    """HTDemucs::separate with a bag of linear models against the oracle's composition
    (same mono-mix statistics fed to both: the driver's are read back from its own normalise)."""
    C, L, seg, sr = 2, 1_000_003, SEG, 44100
    gains = [[0.5, -1.25, 2.0, 1.0], [1.5, 0.0, -0.5, 0.75]][:n_models]
    bag = np.array([[1.0, 1.0, 1.0, 1.0], [0.5, 2.0, 0.0, 1.0]], np.float32)[:n_models]
    mix = synth.sines_plus_pink(31, C, L)
    forward, np_model = gain_model(gains, C, seg, 3, device)
    out = host(stx.htdemucs_separate(dev(mix, device), seg, 4, bag, forward, sample_rate=sr, batch=3,
                                      shifts=shifts, seed=11))
    want = htd.separate(mix, seg, bag, np_model, sample_rate=sr, shifts=shifts, seed=11)
    # The device mono-mix statistics differ from the oracle's sequential sums in the last bits of
    # a double, which can move a normalised sample by one float ulp; everything after is exact.
    assert rel_err(out, want) <= 1e-6


def test_separate_progress_cancel_and_errors(device):
    import torch
    C, L, seg = 1, 50_000, 8_000
    mix = dev(synth.normal(32, (C, L), 0.2), device)
    forward, _ = gain_model([[1.0]], C, seg, 2, device)
    seen = []
    stx.htdemucs_separate(mix, seg, 1, np.ones((1, 1), np.float32), forward, batch=2,
                          progress=lambda d, t: seen.append((d, t)))
    stride, n = stx.htdemucs_split_plan(L, seg, 0.25)
    assert seen == [(d, n) for d in range(1, n + 1)]
    calls = []

    def cancel():
        calls.append(1)
        return len(calls) >= 3
    with pytest.raises(stx.StxError) as e:
        stx.htdemucs_separate(mix, seg, 1, np.ones((1, 1), np.float32), forward, batch=1, should_cancel=cancel)
    assert e.value.status == stx.STATUS_CANCELLED and len(calls) == 3
    with pytest.raises(stx.StxError) as e:
        stx.htdemucs_separate(mix, seg, 1, np.ones((1, 1), np.float32), forward, overlap=1.0)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT and "overlap must be < 1" in e.value.message
