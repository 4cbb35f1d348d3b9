"""GPU parity of the STFT family (stft.hip) against the oracle and the reference's golden vectors.

Bound (north star): SNR >= 110 dB for spectra (the oracle's double spectrum is the reference)
and for STFT -> iSTFT reconstructions, SNR = 10 log10(sum ref^2 / sum err^2)
(tools/stems-parity.cpp:36). Layout changes are exact (bit-identical values).
"""
import glob
import os

import numpy as np
import pytest

import oracle_lib
import stx
import synth
from metrics import snr_db

pytestmark = pytest.mark.gpu

SNR_DB = 110.0
GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "stft_*.npz")))
SPEC_GOLDEN = [p for p in GOLDEN if "torch" in p or "htdemucs" in p]


@pytest.fixture(scope="module")
def orc():
    return oracle_lib.oracle()


_plans = {}


def plan(n):
    if n not in _plans:
        _plans[n] = stx.FFT(n)
    return _plans[n]


def to_dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ws_for(fft, channels, frames, device, use):
    return stx.workspace(stx.istft_workspace_size(fft, channels, frames), device) if use else None


@pytest.mark.parametrize("path", SPEC_GOLDEN, ids=[os.path.basename(p)[5:-4] for p in SPEC_GOLDEN])
@pytest.mark.parametrize("layout", [stx.F_MAJOR, stx.T_MAJOR])
@pytest.mark.parametrize("use_ws", [False, True], ids=["plain", "workspace"])
def test_golden_spectrum_and_inverse(device, path, layout, use_ws):
    d = np.load(path)
    n = int(d["n_fft"])
    x = to_dev(d["x"][None, :], device)
    spec_ref = d["spec"]
    if "torch" in path:
        hop, nm = int(d["hop"]), bool(int(d["normalized"]))
        spec = stx.torch_stft(plan(n), x, hop, nm, layout=layout)
    else:
        spec = stx.htdemucs_spec(plan(n), x, layout=layout)
    got = host(spec)[0]
    if layout == stx.T_MAJOR:
        got = got.T
    assert got.shape == spec_ref.shape
    assert snr_db(got, spec_ref) >= SNR_DB
    # Inverse of the reference spectrum rounded to complex64.
    s = spec_ref.astype(np.complex64)[None]
    sdev = to_dev(s if layout == stx.F_MAJOR else np.ascontiguousarray(s.transpose(0, 2, 1)), device)
    ws = ws_for(plan(n), 1, spec_ref.shape[1], device, use_ws)
    if "torch" in path:
        y = stx.torch_istft(plan(n), sdev, hop, nm, layout=layout, workspace=ws)
    else:
        y = stx.htdemucs_ispec(plan(n), sdev, d["x"].size, layout=layout, workspace=ws)
    y = host(y)[0]
    assert y.shape == d["y"].shape
    assert snr_db(y, d["y"]) >= SNR_DB


def _stereo(seed, length, sigma=0.1):
    return synth.normal(seed, (2, length), sigma)


@pytest.mark.parametrize("use_ws", [False, True], ids=["plain", "workspace"])
def test_htdemucs_spec_c1_full_size(device, orc, use_ws):
    # HTDemucs spec: stereo 343,980 samples, n_fft 4096, hop 1024 -> [2][2048][336].
    length = 343980
    x = _stereo(2024, length)
    f = plan(4096)
    spec = stx.htdemucs_spec(f, to_dev(x, device))
    y = stx.htdemucs_ispec(f, spec, length, workspace=ws_for(f, 2, 336, device, use_ws))
    spec_h, y_h = host(spec), host(y)
    assert spec_h.shape == (2, 2048, 336)
    for c in range(2):
        ref = orc.htdemucs_spec(x[c], 4096)
        assert snr_db(spec_h[c], ref) >= SNR_DB
        yref = orc.htdemucs_ispec(ref, 4096, length)
        assert snr_db(y_h[c], yref) >= SNR_DB


def test_torch_stft_c1_plain_call(device, orc):
    length = 343980
    x = _stereo(2025, length)
    f = plan(4096)
    spec = stx.torch_stft(f, to_dev(x, device), 1024)
    y = stx.torch_istft(f, spec, 1024)
    spec_h, y_h = host(spec), host(y)
    assert spec_h.shape == (2, 2049, 336)
    for c in range(2):
        ref = orc.torch_stft(x[c], 4096, 1024)
        assert snr_db(spec_h[c], ref) >= SNR_DB
        assert snr_db(y_h[c], orc.torch_istft(ref, 4096, 1024)) >= SNR_DB
        assert snr_db(y_h[c], x[c][: y_h.shape[1]]) >= SNR_DB


@pytest.mark.parametrize("normalized", [False, True])
@pytest.mark.parametrize("use_ws", [False, True], ids=["plain", "workspace"])
def test_roformer_stft_c3_full_size(device, orc, normalized, use_ws):
    # RoFormer chunk: stereo 352,800 samples, n_fft 2048, hop 441 -> [2][1025][801] (odd T).
    length = 352800
    x = _stereo(2026, length)
    f = plan(2048)
    spec = stx.torch_stft(f, to_dev(x, device), 441, normalized)
    spec_t = stx.torch_stft(f, to_dev(x, device), 441, normalized, layout=stx.T_MAJOR)
    ws = ws_for(f, 2, 801, device, use_ws)
    y = stx.torch_istft(f, spec, 441, normalized, workspace=ws)
    y_t = stx.torch_istft(f, spec_t, 441, normalized, layout=stx.T_MAJOR, workspace=ws)
    spec_h, spec_th, y_h, y_th = host(spec), host(spec_t), host(y), host(y_t)
    assert spec_h.shape == (2, 1025, 801)
    assert np.array_equal(spec_h, spec_th.transpose(0, 2, 1))
    assert np.array_equal(y_h, y_th)
    for c in range(2):
        ref = orc.torch_stft(x[c], 2048, 441, normalized)
        assert snr_db(spec_h[c], ref) >= SNR_DB
        assert snr_db(y_h[c], orc.torch_istft(ref, 2048, 441, normalized)) >= SNR_DB
        assert snr_db(y_h[c], x[c]) >= SNR_DB


@pytest.mark.parametrize("n", [16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192])
@pytest.mark.parametrize("use_ws", [False, True], ids=["plain", "workspace"])
def test_every_fft_size_stft_round_trip(device, orc, n, use_ws):
    hop = max(1, n // 4 - 1)
    length = 3 * n + 5
    x = _stereo(300 + n, length, 0.5)
    f = plan(n)
    spec = stx.torch_stft(f, to_dev(x, device), hop)
    y = stx.torch_istft(f, spec, hop, workspace=ws_for(f, 2, length // hop + 1, device, use_ws))
    spec_h, y_h = host(spec), host(y)
    for c in range(2):
        ref = orc.torch_stft(x[c], n, hop)
        assert snr_db(spec_h[c], ref) >= SNR_DB
        assert snr_db(y_h[c], orc.torch_istft(ref, n, hop)) >= SNR_DB
    if length > 3 * n // 8 * 2:
        s2 = stx.htdemucs_spec(f, to_dev(x, device))
        y2 = stx.htdemucs_ispec(f, s2, length, workspace=ws_for(f, 2, s2.shape[2], device, use_ws))
        s2h, y2h = host(s2), host(y2)
        for c in range(2):
            ref = orc.htdemucs_spec(x[c], n)
            assert snr_db(s2h[c], ref) >= SNR_DB
            assert snr_db(y2h[c], orc.htdemucs_ispec(ref, n, length)) >= SNR_DB


# Every power of two st::FFT accepts (src/stft.h:21-22): 2, 4, 8 as register transforms, 16 to
# 8192 as LDS kernels, and above 8192 in four steps (n1 x n2 transforms around transposes).
@pytest.mark.parametrize("n", [2, 4, 8, 16, 256, 2048, 4096, 8192, 16384, 32768, 1 << 20])
def test_fft_run_against_oracle(device, orc, n):
    import torch
    v = synth.normal(n, (3, 2 * n), 1.0).astype(np.float64)
    a = v[:, 0::2] + 1j * v[:, 1::2]
    d = to_dev(a.astype(np.complex64), device)
    plan(n).run(d)
    fw = host(d)
    plan(n).run(d, inverse=True)
    back = host(d) / n
    for b in range(3):
        assert snr_db(fw[b], orc.fft(a[b].astype(np.complex64).astype(np.complex128))) >= SNR_DB
        assert snr_db(back[b], a[b].astype(np.complex64)) >= SNR_DB
    del torch


def test_fft_run_only_sizes_have_no_stft(device):
    """Sizes with only a complex transform (2, 4, 8 and above 8192) report UNSUPPORTED for the
    STFT/iSTFT; the reference never frames at those sizes."""
    import torch
    x = torch.zeros((1, 100000), dtype=torch.float32, device=device)
    for n in (8, 16384):
        f = plan(n)
        assert f.size() == n
        with pytest.raises(stx.StxError) as e:
            stx.torch_stft(f, x, n // 4)
        assert e.value.status == stx.STATUS_UNSUPPORTED


def test_fft_impulse_known_answer(device):
    n = 2048
    a = np.zeros((1, n), np.complex64)
    a[0, 7] = 1.0
    d = to_dev(a, device)
    plan(n).run(d)
    k = np.arange(n)
    assert np.max(np.abs(host(d)[0] - np.exp(-2j * np.pi * 7 * k / n))) < 1e-6


def test_stft_errors(device):
    import torch
    x = torch.zeros((1, 1024), dtype=torch.float32, device=device)
    with pytest.raises(stx.StxError) as e:
        stx.torch_stft(plan(2048), x, 441)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR
    with pytest.raises(stx.StxError) as e:
        stx.htdemucs_spec(plan(4096), x)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR


def test_small_hop_needs_several_rounds(device, orc):
    # hop n/64 makes every output tile overlap 64 frames, twice the 32 one workgroup transforms
    # at once at n_fft 1024, so the fused path loops over rounds.
    n, hop, length = 1024, 16, 4000
    x = _stereo(55, length, 0.3)
    f = plan(n)
    spec = stx.torch_stft(f, to_dev(x, device), hop)
    y = host(stx.torch_istft(f, spec, hop))
    spec_h = host(spec)
    for c in range(2):
        ref = orc.torch_stft(x[c], n, hop)
        assert snr_db(spec_h[c], ref) >= SNR_DB
        assert snr_db(y[c], orc.torch_istft(ref, n, hop)) >= SNR_DB


@pytest.mark.parametrize("layout", [stx.F_MAJOR, stx.T_MAJOR])
@pytest.mark.parametrize("n,hop,length,channels,sub", [
    (2048, 441, 352800, 48, 3),     # 48 RoFormer chunks: 3,216 tiles; 3 chunks: 201 tiles
    (1024, 8, 2000, 8, 1),          # 4 rounds of 32 frames per tile: 2,000 tiles; 1 channel: 250
])
def test_istft_more_tiles_than_resident_workgroups(device, orc, layout, n, hop, length, channels, sub):
    # A batch whose tiles outnumber the workgroups the GPU holds at once: each workgroup takes
    # several tiles (and prefetches the next tile's frames). Every channel must equal, bit for
    # bit, the same channels inverted in a call small enough to give each tile its own workgroup.
    x = synth.normal(4100 + n, (channels, length), 0.2)
    f = plan(n)
    spec = stx.torch_stft(f, to_dev(x, device), hop, layout=layout)
    y = host(stx.torch_istft(f, spec, hop, layout=layout))
    for i in range(0, channels, sub):
        part = host(stx.torch_istft(f, spec[i:i + sub].contiguous(), hop, layout=layout))
        assert np.array_equal(part, y[i:i + sub]), f"channels {i}..{i + sub - 1}"
    spec_h = host(spec)
    for c in (0, channels - 1):
        s = spec_h[c] if layout == stx.F_MAJOR else spec_h[c].T
        ref = orc.torch_stft(x[c], n, hop)
        assert snr_db(s, ref) >= SNR_DB
        assert snr_db(y[c], orc.torch_istft(ref, n, hop)) >= SNR_DB


@pytest.mark.parametrize("layout", [stx.F_MAJOR, stx.T_MAJOR])
def test_htdemucs_ispec_many_segments_same_bits_as_pairs(device, orc, layout):
    # 16 HTDemucs segments (n_fft 4096) in one call: 8-frame tiles of 5 hops, 1,088 of them,
    # several per workgroup; a call of two segments takes 6-frame tiles of 3 hops, one per
    # workgroup. Each sample adds the same frames in the same order either way, so every
    # channel must come out bit for bit the same.
    length, channels = 343980, 16
    x = synth.normal(4242, (channels, length), 0.1)
    f = plan(4096)
    spec = stx.htdemucs_spec(f, to_dev(x, device), layout=layout)
    y = host(stx.htdemucs_ispec(f, spec, length, layout=layout))
    for i in range(0, channels, 2):
        part = host(stx.htdemucs_ispec(f, spec[i:i + 2].contiguous(), length, layout=layout))
        assert np.array_equal(part, y[i:i + 2]), f"channels {i}, {i + 1}"
    spec_h = host(spec)
    for c in (0, channels - 1):
        s = spec_h[c] if layout == stx.F_MAJOR else spec_h[c].T
        ref = orc.htdemucs_spec(x[c], 4096)
        assert snr_db(s, ref) >= SNR_DB
        assert snr_db(y[c], orc.htdemucs_ispec(ref, 4096, length)) >= SNR_DB


def test_istft_many_tiles_graph_replays(device):
    """A captured torch_istft call whose tiles outnumber the resident workgroups, replayed on new
    spectra with eager work between the replays: every replay equals the eager call's bits."""
    import torch
    n, hop, length, channels = 2048, 441, 352800, 24
    f = plan(n)
    x = to_dev(synth.normal(4300, (channels, length), 0.2), device)
    spec = stx.torch_stft(f, x, hop)
    y = torch.empty((channels, length), device=device)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        stx.torch_istft(f, spec, hop, out=y, stream=s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            stx.torch_istft(f, spec, hop, out=y, stream=s)
    torch.cuda.synchronize()
    for rep in range(3):
        xn = to_dev(synth.normal(4310 + rep, (channels, length), 0.1 + 0.2 * rep), device)
        spec.copy_(stx.torch_stft(f, xn, hop))
        want = host(stx.torch_istft(f, spec, hop))
        g.replay()
        assert np.array_equal(host(y), want), f"replay {rep}"


@pytest.mark.parametrize("trim", [0, 4999])
def test_htdemucs_ispec_many_segments_trimmed(device, orc, trim):
    # The batched call with an output shorter than the segment (the tiles' last one cut short)
    # against one segment at a time.
    length, channels = 343980, 12
    x = synth.normal(4400 + trim, (channels, length), 0.1)
    f = plan(4096)
    spec = stx.htdemucs_spec(f, to_dev(x, device))
    y = host(stx.htdemucs_ispec(f, spec, length - trim))
    for i in range(channels):
        one = host(stx.htdemucs_ispec(f, spec[i:i + 1].contiguous(), length - trim))
        assert np.array_equal(one, y[i:i + 1]), f"channel {i}"
    ref = orc.htdemucs_spec(x[channels - 1], 4096)
    assert snr_db(y[channels - 1], orc.htdemucs_ispec(ref, 4096, length - trim)) >= SNR_DB


def test_workspace_too_small(device):
    f = plan(2048)
    x = to_dev(_stereo(56, 20000), device)
    spec = stx.torch_stft(f, x, 441)
    ws = stx.workspace(stx.istft_workspace_size(f, 2, spec.shape[2]) - 4096, device)
    with pytest.raises(stx.StxError) as e:
        stx.torch_istft(f, spec, 441, workspace=ws)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT


# ----------------------------------------- st::VRFFT sizes (mixed-radix kernels on the device)
_any_plans = {}


def any_plan(n):
    if n not in _any_plans:
        _any_plans[n] = stx.FFT(n, any_size=True)
    return _any_plans[n]


@pytest.mark.parametrize("n", [7680, 3840, 960, 640, 320, 480, 6000])
def test_fft_run_any_size(device, orc, n):
    """Complex transforms of VRFFT's sizes against the oracle's Bluestein (src/vr_dsp.h:11-37)."""
    v = synth.normal(n + 1, (3, 2 * n), 1.0).astype(np.float64)
    a = (v[:, 0::2] + 1j * v[:, 1::2]).astype(np.complex64)
    d = to_dev(a, device)
    any_plan(n).run(d)
    fw = host(d)
    any_plan(n).run(d, inverse=True)
    back = host(d) / n
    for b in range(3):
        assert snr_db(fw[b], orc.vrfft(a[b].astype(np.complex128))) >= SNR_DB
        assert snr_db(back[b], a[b]) >= SNR_DB


@pytest.mark.parametrize("layout", [stx.F_MAJOR, stx.T_MAJOR])
@pytest.mark.parametrize("normalized", [False, True])
def test_torch_stft_7680_kim_chunk(device, orc, layout, normalized):
    """Kim_Vocal_2's transform (src/tfc_tdf.cpp:355-359): n_fft 7680, hop 1024, one chunk of
    1024 x 255 = 261,120 stereo samples -> [2][3841][256]; STFT and the workspace iSTFT."""
    length, n, hop = 261120, 7680, 1024
    x = _stereo(7680, length)
    f = any_plan(n)
    spec = stx.torch_stft(f, to_dev(x, device), hop, normalized, layout=layout)
    ws = stx.workspace(stx.istft_workspace_size(f, 2, length // hop + 1), device)
    y = stx.torch_istft(f, spec, hop, normalized, layout=layout, workspace=ws)
    spec_h, y_h = host(spec), host(y)
    if layout == stx.T_MAJOR:
        spec_h = spec_h.transpose(0, 2, 1)
    assert spec_h.shape == (2, 3841, 256)
    for c in range(2):
        ref = orc.torch_stft(x[c], n, hop, normalized)
        assert snr_db(spec_h[c], ref) >= SNR_DB
        assert snr_db(y_h[c], orc.torch_istft(ref, n, hop, normalized)) >= SNR_DB
    # A workspace only 4-byte aligned (the frames are then stored a float at a time): same bits.
    ws_odd = stx.workspace(stx.istft_workspace_size(f, 2, length // hop + 1) + 4, device)[1:]
    y_odd = host(stx.torch_istft(f, spec, hop, normalized, layout=layout, workspace=ws_odd))
    assert np.array_equal(y_odd, y_h)


@pytest.mark.parametrize("n,hop", [(320, 80), (640, 160), (960, 240), (1536, 256)])
@pytest.mark.parametrize("extra", [3, "hop"])
def test_torch_stft_vr_sizes_round_trip(device, orc, n, hop, extra):
    """An odd frame count (length 20 n + 3) and an even one (20 n + hop): the f-major iSTFT
    transforms two frames per block when the count is even."""
    length = 20 * n + (hop if extra == "hop" else extra)
    x = _stereo(n, length, 0.5)
    f = any_plan(n)
    spec = stx.torch_stft(f, to_dev(x, device), hop)
    ws = stx.workspace(stx.istft_workspace_size(f, 2, length // hop + 1), device)
    y = stx.torch_istft(f, spec, hop, workspace=ws)
    spec_h, y_h = host(spec), host(y)
    for c in range(2):
        ref = orc.torch_stft(x[c], n, hop)
        assert snr_db(spec_h[c], ref) >= SNR_DB
        assert snr_db(y_h[c], orc.torch_istft(ref, n, hop)) >= SNR_DB


@pytest.mark.parametrize("n,hop,frames", [(960, 240, 82), (7680, 1024, 32)])
def test_mixed_pairs_unaligned_spectrum(device, n, hop, frames):
    """The mixed-radix STFT and iSTFT transform two f-major frames per block when the frame count
    is even and the spectrum 16-byte aligned; a spectrum 8 bytes off that takes one frame per
    block. Both give the same bits (the run-time plan at 960 and the compiled one at 7680)."""
    import torch
    length = (frames - 1) * hop
    x = to_dev(_stereo(n, length, 0.5), device)
    f = any_plan(n)
    F, T = n // 2 + 1, length // hop + 1
    assert T == frames
    a = stx.torch_stft(f, x, hop)
    assert a.data_ptr() % 16 == 0
    buf = torch.empty(2 * 2 * F * T + 2, dtype=torch.float32, device=x.device)
    b = buf[2:].view(torch.complex64).view(2, F, T)
    assert b.data_ptr() % 16 == 8
    stx.torch_stft(f, x, hop, out=b)
    assert np.array_equal(host(a), host(b))
    ws = stx.workspace(stx.istft_workspace_size(f, 2, T), device)
    ya = host(stx.torch_istft(f, a, hop, workspace=ws))
    yb = host(stx.torch_istft(f, b, hop, workspace=ws))
    assert np.array_equal(ya, yb)


def test_any_size_errors(device):
    import torch
    for n in (7, 14, 22, 20000):
        with pytest.raises(stx.StxError) as e:
            stx.FFT(n, any_size=True)
        assert e.value.status == stx.STATUS_UNSUPPORTED
    with pytest.raises(stx.StxError) as e:
        stx.FFT(7680)                                              # st::FFT: powers of two only
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    assert any_plan(2048).n == 2048                                 # a power of two: the radix-16 plan
    f = any_plan(7680)
    x = torch.zeros((1, 20000), dtype=torch.float32, device=device)
    spec = stx.torch_stft(f, x, 1024)
    with pytest.raises(stx.StxError) as e:
        stx.torch_istft(f, spec, 1024)                             # needs the workspace variant
    assert e.value.status == stx.STATUS_UNSUPPORTED
    with pytest.raises(stx.StxError) as e:
        stx.htdemucs_spec(f, x)
    assert e.value.status == stx.STATUS_UNSUPPORTED
