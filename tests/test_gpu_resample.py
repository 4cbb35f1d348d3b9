"""GPU parity of the resampler (resample.hip) against the oracle (src/audio.h:17-59).

Bars: the per-tap kernel (STX_RESAMPLE_EXACT=1) is bit-exact (the device sums the reference's
double products in the reference's order over a table computed by the reference's formula);
the default phase-table kernel, whose weights come from the output's exact rational position
instead of the reference's rounded one, has SNR >= 110 dB and every sample within 1e-6 of the
output's rms. A rate pair whose staged input tile exceeds the device's LDS per workgroup
(44.1 -> 8 kHz here: 210 KB) takes the per-tap kernel by default and is bit-exact either way.
Shapes: a 180 s stereo song at 48 kHz to the models' 44.1 kHz, and short inputs for other rate
pairs, mono, stereo and 3 channels.
"""
import numpy as np
import pytest

import oracle_lib
import stx
import synth
from metrics import snr_db

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rs():
    return oracle_lib.resample()


def dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("src,dst,C,n", [(48000, 44100, 2, 8640000), (22050, 44100, 2, 30001), (44100, 16000, 1, 44100),
                                         (96000, 44100, 3, 9601), (44100, 48000, 2, 100), (8000, 44100, 1, 37),
                                         (44100, 8000, 2, 20001), (48000, 44100, 2, 1), (44100, 48000, 1, 2),
                                         (22050, 44100, 1, 1)])
def test_resample_parity(device, rs, src, dst, C, n, monkeypatch):
    x = synth.sines_plus_pink(src % 1000, C, n) if n > 1000 else synth.normal(src % 1000, (C, n), 0.3)
    r = stx.Resampler(src, dst)
    xd = dev(x, device)
    want = rs(x, src, dst)
    got = host(r(xd))
    assert got.shape == want.shape and r.length(n) == want.shape[1]
    # A filter's output: SNR >= 110 dB, and every sample within 1e-6 of the signal's rms (measured
    # 167 dB and 2.0e-7 rms for the 180 s song). An elementwise relative bound does not apply:
    # outputs that cancel to near zero carry the weights' 1e-9 difference times the inputs' scale.
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert snr_db(got, want) >= 110.0
    assert float(np.max(np.abs(got.astype(np.float64) - want))) <= 1e-6 * rms
    monkeypatch.setenv("STX_RESAMPLE_EXACT", "1")
    exact = host(r(xd))
    assert np.array_equal(exact, want)


@pytest.mark.parametrize("src,dst,C,n", [(48000, 44100, 2, 48001), (44100, 48000, 1, 44101), (22050, 44100, 2, 3001),
                                         (96000, 44100, 3, 9601)])
def test_resample_nonfinite(device, rs, src, dst, C, n, monkeypatch):
    """NaN, +inf and -inf samples (NaN at each end) reach exactly the outputs whose window holds
    them in the reference (src/audio.h:44-52): the phase kernel's pair loop sums a tap only where
    its own phase's window has it, so the NaN and infinite outputs are the oracle's and the finite
    outputs keep the usual bound; the per-tap kernel is bit-identical, NaNs included.

    An infinite output's sign is its tap's weight's. At a zero of the kernel the reference's weight
    and the exact phase's are both below 1e-14 and may differ in sign (a restatement of both
    weight formulas finds 2, 0, 0 and 3 such taps for these cases), so up to one sign per infinite
    input sample may differ."""
    x = synth.normal(src % 997, (C, n), 0.3)
    for c in range(C):
        x[c, [0, n // 3 + c, n // 2 + 7 * c, n - 1]] = [np.nan, np.inf, -np.inf, np.nan]
    r = stx.Resampler(src, dst)
    xd = dev(x, device)
    want = rs(x, src, dst)
    got = host(r(xd))
    assert np.isnan(want).any() and np.isinf(want).any()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf)
    assert int(np.sum(np.sign(got[inf]) != np.sign(want[inf]))) <= 2 * C     # 2 infinite samples per channel
    fin = np.isfinite(want)
    rms = float(np.sqrt(np.mean(want[fin].astype(np.float64) ** 2)))
    assert float(np.max(np.abs(got[fin].astype(np.float64) - want[fin]))) <= 1e-6 * rms
    monkeypatch.setenv("STX_RESAMPLE_EXACT", "1")
    assert np.array_equal(host(r(xd)), want, equal_nan=True)


def test_equal_rates_copy(device):
    x = synth.normal(3, (2, 1000), 1.0)
    r = stx.Resampler(44100, 44100)
    assert r.length(1000) == 1000
    assert np.array_equal(host(r(dev(x, device))), x)


def test_errors(device):
    with pytest.raises(stx.StxError):
        stx.Resampler(0, 44100)
    import torch
    r = stx.Resampler(48000, 44100)
    with pytest.raises(stx.StxError) as e:
        r(torch.zeros((9, 100), device=device))
    assert e.value.status == stx.STATUS_UNSUPPORTED
