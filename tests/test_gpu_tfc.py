"""GPU parity of the TFC-TDF chunking (demix.hip with MSST rules, tfc.hip) against the oracle.

MSST chunk inputs and overlap-add, UVR chunk inputs and overlap-add are bit-exact with the oracle
for identical model outputs (double products and sums in chunk order, one division). The driver
(stx_tfc_tdf_separate, TFCTDF::separate) is checked with per-stem-gain models for both chunkings,
with compensation and the complement stem, bit-exact, and for its error codes.

Shapes: the 180 s stereo song at an MDX-Net chunk of hop 1024 x (dim_t 256 - 1) = 261,120
samples: MSST with num_overlap 4 (step 65,280), UVR at n_fft 7680 (Kim_Vocal_2; step 253,440)
and at overlap 0.5; plus small and ragged geometries.
"""
import numpy as np
import pytest

import oracle_lib
import stx
import synth
from hip_util import d2d

pytestmark = pytest.mark.gpu

SONG, CHUNK = 7938000, 261120


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


MSST_CASES = [(SONG, CHUNK, CHUNK // 4), (1000, 100, 25), (1000, 100, 100), (150, 100, 25), (1001, 97, 31),
              (60, 100, 50), (5003, 64, 9), (351, 100, 100)]


@pytest.mark.parametrize("length,chunk,step", MSST_CASES)
def test_msst_chunks_and_ola_bit_exact(device, od, length, chunk, step):
    mix = synth.normal(length % 1000 + 5, (2, length), 0.3)
    plan = stx.Demix(length, 2, chunk, step, rules=stx.DEMIX_MSST)
    parts = host(plan.chunks(dev(mix, device)))
    assert np.array_equal(parts, od.msst_chunks(mix, chunk, step))
    S = 1 if length > 1000000 else 3
    y = synth.uniform(length % 977, (plan.n_chunks, S, 2, chunk))
    got = host(plan.overlap_add(dev(y, device)))
    assert np.array_equal(got, od.msst_ola(y, length, chunk, step))


def test_msst_plan_and_window(device, od):
    geom, table = stx.demix_plan(1000, 100, 25, rules=stx.DEMIX_MSST)
    assert geom["n_chunks"] == od.L.orc_msst_n_chunks(1000, 100, 25)
    # Only the chunk after which the loop ends keeps full weight at its end.
    assert list(table["fade_out"]).count(0) == 1 and table["fade_out"][-1] == 0
    assert np.array_equal(stx.demix_window(100, rules=stx.DEMIX_MSST), od.msst_window(100))


UVR_CASES = [(SONG, CHUNK, 7680, -1.0), (SONG, CHUNK, 7680, 0.5), (SONG, CHUNK, 7680, 0.0), (5000, 512, 128, -1.0),
             (300, 512, 128, -1.0), (4099, 600, 100, 0.25), (4099, 600, 100, 0.8)]


@pytest.mark.parametrize("length,chunk,n_fft,overlap", UVR_CASES)
def test_uvr_chunks_and_ola_bit_exact(device, od, length, chunk, n_fft, overlap, monkeypatch):
    """Chunks and overlap-add against the oracle, bit for bit; the overlap-add with 32-bit
    indices (every case here) and with 64-bit ones (STX_UVR_WIDE_INDEX=1) alike."""
    mix = synth.normal(length % 1000 + 7, (2, length), 0.3)
    plan = stx.UvrDemix(length, 2, chunk, n_fft, overlap)
    n, M, step = od.uvr_geometry(length, chunk, n_fft, overlap)
    assert (plan.n_chunks, plan.padded_len, plan.step) == (n, M, step)
    parts = host(plan.chunks(dev(mix, device)))
    assert np.array_equal(parts, od.uvr_chunks(mix, chunk, n_fft, overlap))
    S = 1 if length > 1000000 else 3
    y = synth.uniform(length % 991, (n, S, 2, chunk))
    yd = dev(y, device)
    got = host(plan.overlap_add(yd))
    assert np.array_equal(got, od.uvr_ola(y, length, chunk, n_fft, overlap))
    monkeypatch.setenv("STX_UVR_WIDE_INDEX", "1")
    assert np.array_equal(host(plan.overlap_add(yd)), got)


def test_uvr_ola_non_finite_outputs(device, od):
    """Model outputs holding inf, -inf and NaN: the overlap-add divides by the weight sum as the
    reference does (src/tfc_tdf.cpp:427, no nan_to_num), so an infinite sum stays infinite (the
    correctly rounded quotient's residual would be inf - inf) and NaN stays NaN."""
    length, chunk, n_fft, overlap = 5000, 512, 128, -1.0
    plan = stx.UvrDemix(length, 2, chunk, n_fft, overlap)
    y = synth.uniform(31, (plan.n_chunks, 2, 2, chunk))
    y[1, 0, 0, 100] = np.inf
    y[2, 1, 1, 7] = -np.inf
    y[3, 0, 1, 300] = np.nan
    assert plan.step == 384
    y[4, 1, 0, 450] = np.inf
    y[5, 1, 0, 450 - 384] = -np.inf                     # the same sample from two chunks: inf - inf
    got = host(plan.overlap_add(dev(y, device)))
    want = od.uvr_ola(y, length, chunk, n_fft, overlap)
    assert np.isposinf(got).any() and np.isneginf(got).any() and np.isnan(got).any()
    assert np.array_equal(got, want, equal_nan=True)


def test_uvr_ola_extreme_magnitudes(device, od):
    """Where one chunk covers a sample with a non-zero weight, the kernel copies the model's value
    (the reference's (0 + y w) / (0 + w) rounds back to y); checked bit for bit at the float
    extremes: subnormals down to 2^-149, values up to 3.4e38, signed zeros and non-finite values,
    in single-cover samples and in the overlaps."""
    length, chunk, n_fft, overlap = 20000, 2048, 512, -1.0
    plan = stx.UvrDemix(length, 2, chunk, n_fft, overlap)
    rng = np.random.default_rng(5)
    y = synth.uniform(41, (plan.n_chunks, 2, 2, chunk))
    y *= np.exp2(rng.integers(-149, 127, y.shape)).astype(np.float32)
    flat = y.reshape(-1)
    idx = rng.choice(flat.size, 64, replace=False)
    flat[idx[:16]] = np.float32(2.0 ** -149)
    flat[idx[16:24]] = -0.0
    flat[idx[24:32]] = np.float32(3.4e38)
    flat[idx[32:36]] = np.inf
    flat[idx[36:40]] = np.nan
    got = host(plan.overlap_add(dev(y, device)))
    want = od.uvr_ola(y, length, chunk, n_fft, overlap)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    m = ~np.isnan(got)
    assert np.array_equal(got[m].view(np.uint32), want[m].view(np.uint32))          # signed zeros too


def test_uvr_errors(device):
    with pytest.raises(stx.StxError) as e:
        stx.UvrDemix(1000, 2, 100, 128)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR and "chunk shorter than the FFT" in e.value.message
    with pytest.raises(stx.StxError) as e:
        stx.UvrDemix(1000, 2, 512, 128, 1.0)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT and "overlap too large" in e.value.message


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


@pytest.mark.parametrize("chunking", [stx.TFC_MSST, stx.TFC_UVR])
@pytest.mark.parametrize("complement,compensate", [(False, 1.0), (True, 1.035)])
def test_separate_gains_bit_exact(device, od, chunking, complement, compensate):
    C, L, chunk, n_fft = 2, 300007, 16384, 4096
    gains = [0.5, -1.25]
    mix = synth.sines_plus_pink(12, C, L)
    out = host(stx.tfc_tdf_separate(dev(mix, device), chunk, n_fft, chunking, 2,
                                    gains_separator(gains, C, chunk, 3, device), num_overlap=4,
                                    compensate=compensate, complement=complement, batch=3))
    g = np.array(gains, np.float32)[None, :, None, None]
    if chunking == stx.TFC_MSST:
        step = stx.demix_step(chunk, 4)
        est = od.msst_ola(g * od.msst_chunks(mix, chunk, step)[:, None], L, chunk, step)
    else:
        est = od.uvr_ola(g * od.uvr_chunks(mix, chunk, n_fft)[:, None], L, chunk, n_fft)
    want = od.tfc_post(mix, est, compensate, complement)
    assert np.array_equal(out, want)


def test_separate_errors_and_cancel(device):
    import torch
    C, L, chunk = 2, 20000, 4096
    sep = gains_separator([1.0], C, chunk, 2, device)
    mix = synth.normal(13, (C, L), 0.2)
    bad = mix.copy()
    bad[1, 777] = np.inf
    with pytest.raises(stx.StxError) as e:
        stx.tfc_tdf_separate(dev(bad, device), chunk, 1024, stx.TFC_MSST, 1, sep)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR and "non-finite" in e.value.message
    with pytest.raises(stx.StxError) as e:
        stx.tfc_tdf_separate(dev(mix, device), chunk, 1024, stx.TFC_MSST, 1, sep, shifts=1)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR and "shifts" in e.value.message
    with pytest.raises(stx.StxError) as e:
        stx.tfc_tdf_separate(dev(mix, device), chunk, 1024, stx.TFC_UVR, 1, sep, overlap=1.0)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    with pytest.raises(stx.StxError) as e:
        stx.tfc_tdf_separate(dev(mix, device), 1000, 1024, stx.TFC_UVR, 1, gains_separator([1.0], C, 1000, 2, device))
    assert e.value.status == stx.STATUS_RUNTIME_ERROR and "shorter than the FFT" in e.value.message
    calls, seen = [], []

    def cancel():
        calls.append(1)
        return len(calls) >= 3
    with pytest.raises(stx.StxError) as e:
        stx.tfc_tdf_separate(dev(mix, device), chunk, 1024, stx.TFC_UVR, 1, sep, batch=1, should_cancel=cancel)
    assert e.value.status == stx.STATUS_CANCELLED and len(calls) == 3
    stx.tfc_tdf_separate(dev(mix, device), chunk, 1024, stx.TFC_MSST, 1, sep, batch=2,
                         progress=lambda d, t: seen.append((d, t)))
    n = stx.Demix(L, C, chunk, stx.demix_step(chunk, 4), rules=stx.DEMIX_MSST).n_chunks
    assert seen == [(d, n) for d in range(1, n + 1)]
