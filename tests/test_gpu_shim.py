"""The drop-in C++ shim (include/stx_st.hpp: st::FFT, htdemucs_spec/ispec, torch_stft/istft with
the signatures of src/stft.h) against the oracle, on host buffers as the reference's callers
pass them (src/htdemucs.cpp:428,470, src/roformer.cpp:223,279). Same bound as the device
entry points: SNR >= 110 dB for spectra and reconstructions; the reference's exceptions."""
import numpy as np
import pytest

import oracle_lib
import shim_lib
import synth
from metrics import snr_db

pytestmark = pytest.mark.gpu

SNR_DB = 110.0


@pytest.fixture(scope="module")
def orc():
    return oracle_lib.oracle()


def test_shim_htdemucs_round_trip_c1(device, orc):
    x = synth.normal(11, (343980,), 0.1)
    rc, spec = shim_lib.htdemucs_spec(x, 4096)
    assert rc == 0 and spec.shape == (2048, 336)
    want = orc.htdemucs_spec(x, 4096)
    assert snr_db(spec, want) >= SNR_DB
    rc, y = shim_lib.htdemucs_ispec(want, 4096, x.size)
    assert rc == 0
    assert snr_db(y, orc.htdemucs_ispec(want, 4096, x.size)) >= SNR_DB


@pytest.mark.parametrize("normalized", [False, True])
def test_shim_torch_round_trip_c3(device, orc, normalized):
    x = synth.normal(12, (352800,), 0.1)
    rc, spec = shim_lib.torch_stft(x, 2048, 441, normalized)
    assert rc == 0 and spec.shape == (1025, 801)
    want = orc.torch_stft(x, 2048, 441, normalized)
    assert snr_db(spec, want) >= SNR_DB
    rc, y = shim_lib.torch_istft(want, 2048, 441, normalized)
    assert rc == 0
    assert snr_db(y, orc.torch_istft(want, 2048, 441, normalized)) >= SNR_DB


@pytest.mark.parametrize("n", [2, 8, 16, 1024, 4096, 16384])
def test_shim_fft(device, orc, n):
    a = (synth.normal(n, (3, n), 1.0) + 1j * synth.normal(n + 1, (3, n), 1.0)).astype(np.complex128)
    for inverse in (False, True):
        rc, got = shim_lib.fft(a, inverse)
        assert rc == 0
        want = np.stack([orc.fft(row, inverse) for row in a])
        assert snr_db(got, want) >= SNR_DB


def test_shim_fft_transforms_exactly_n_points(device, orc):
    """src/stft.h:35-49 transforms a[0..n) and leaves the rest of the vector alone."""
    n, extra = 1024, 77
    a = (synth.normal(5, (n + extra,), 1.0) + 1j * synth.normal(6, (n + extra,), 1.0)).astype(np.complex128)
    for inverse in (False, True):
        rc, got = shim_lib.fft_prefix(a, n, inverse)
        assert rc == 0
        assert snr_db(got[:n], orc.fft(a[:n], inverse)) >= SNR_DB
        assert np.array_equal(got[n:], a[n:])
    assert shim_lib.lib().shim_fft_run_short(n) == 1          # shorter than n: std::invalid_argument


def test_shim_exceptions(device):
    L = shim_lib.lib()
    assert L.shim_fft_create(3) == 1                 # std::invalid_argument, like src/stft.h:22
    assert L.shim_istft_short_spectrum(2048) == 1
    x = np.zeros(100, np.float32)
    rc, _ = shim_lib.torch_stft(x, 2048, 441)       # reflect pad larger than the signal
    assert rc == 2                                   # std::runtime_error, like src/stft.h:59
