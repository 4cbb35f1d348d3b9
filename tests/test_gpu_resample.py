"""GPU parity of the resampler (resample.hip) against the oracle (src/audio.h:17-59).

Bar: bit-exact (the device sums the reference's double products in the reference's order over
a table computed by the reference's formula). Shapes: a 180 s stereo song at 48 kHz to the
models' 44.1 kHz, and short inputs for other rate pairs, mono and 3 channels.
"""
import numpy as np
import pytest

import oracle_lib
import stx
import synth

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
                                         (96000, 44100, 3, 9601), (44100, 48000, 2, 100), (8000, 44100, 1, 37)])
def test_resample_bit_exact(device, rs, src, dst, C, n):
    x = synth.sines_plus_pink(src % 1000, C, n) if n > 1000 else synth.normal(src % 1000, (C, n), 0.3)
    r = stx.Resampler(src, dst)
    got = host(r(dev(x, device)))
    want = rs(x, src, dst)
    assert got.shape == want.shape and r.length(n) == want.shape[1]
    assert np.array_equal(got, want)


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
