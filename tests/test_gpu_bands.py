"""GPU parity of the band path (bands.hip) against the oracle.

Band gather and scatter-average + apply are compared bit for bit with the oracle fed the same
complex64 spectrum (both accumulate the masks in double in the reference's order and round
once). The whole RoFormer spectral path on one 8 s stereo chunk (STFT 2048/441 -> band gather
-> seeded masks -> scatter-average + apply -> iSTFT) is compared with the oracle's double
path at SNR >= 110 dB per stem and channel (tools/stems-parity.cpp:36).
"""
import numpy as np
import pytest

import oracle_lib
import stx
import synth
from metrics import rel_err, snr_db

pytestmark = pytest.mark.gpu

SR, NFFT, HOP, NMELS = 44100, 2048, 441, 60
BS_FPB = [2] * 24 + [4] * 12 + [12] * 8 + [24] * 8 + [48] * 8 + [128, 129]


@pytest.fixture(scope="module")
def ob():
    return oracle_lib.bands()


@pytest.fixture(scope="module")
def mel():
    return stx.mel_band_map(SR, NFFT, NMELS)


def dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rand_spec(seed, batch, C, F, T):
    v = synth.normal(seed, (2, batch, C, F, T), 1.0)
    return (v[0] + 1j * v[1]).astype(np.complex64)            # [batch][C][F][T]


@pytest.mark.parametrize("kind", ["mel", "bs"])
@pytest.mark.parametrize("layout", [stx.F_MAJOR, stx.T_MAJOR])
def test_gather_bit_exact(device, ob, mel, kind, layout):
    sizes, freqs = mel if kind == "mel" else (np.array(BS_FPB, np.int32), np.arange(1025, dtype=np.int32))
    C, F, T, batch = 2, 1025, 801, 2
    z = rand_spec(11, batch, C, F, T)
    bands = stx.Bands(sizes, freqs, F, C)
    zd = z if layout == stx.F_MAJOR else np.ascontiguousarray(z.transpose(0, 1, 3, 2))
    feat = host(bands.gather(dev(zd, device), T, layout=layout))
    assert feat.shape == (batch, int(sizes.sum()) * C * 2 * T)
    for b in range(batch):
        assert np.array_equal(feat[b], ob.gather(sizes, freqs, z[b].astype(np.complex128)))


@pytest.mark.parametrize("kind", ["mel", "bs"])
@pytest.mark.parametrize("layout", [stx.F_MAJOR, stx.T_MAJOR])
@pytest.mark.parametrize("S,zero_dc", [(1, False), (4, True)])
def test_scatter_apply_bit_exact(device, ob, mel, kind, layout, S, zero_dc):
    sizes, freqs = mel if kind == "mel" else (np.array(BS_FPB, np.int32), np.arange(1025, dtype=np.int32))
    C, F, T, batch = 2, 1025, 801 if S == 1 else 97, 2
    z = rand_spec(12, batch, C, F, T)
    tf = int(sizes.sum()) * C * 2
    masks = synth.uniform(13, (batch, S, tf * T))
    bands = stx.Bands(sizes, freqs, F, C)
    zd = z if layout == stx.F_MAJOR else np.ascontiguousarray(z.transpose(0, 1, 3, 2))
    out = host(bands.scatter_apply(dev(masks, device), dev(zd, device), T, layout=layout, zero_dc=zero_dc))
    if layout == stx.T_MAJOR:
        out = out.transpose(0, 1, 2, 4, 3)
    for b in range(batch):
        ref = ob.scatter_apply(sizes, freqs, masks[b], z[b].astype(np.complex128), zero_dc)
        assert np.array_equal(out[b], ref.astype(np.complex64))


def test_scatter_apply_non_finite_masks(device, ob, mel):
    """Masks holding inf and NaN (a diverged model): the average of a bin's band values divides
    by the band count like the reference (src/roformer.cpp:270-275), inf stays inf, NaN stays
    NaN, and the complex multiply follows; the same bits as the oracle, NaNs in place."""
    sizes, freqs = mel
    C, F, T = 2, 1025, 33
    z = rand_spec(14, 1, C, F, T)[0]
    tf = int(sizes.sum()) * C * 2
    masks = synth.uniform(15, (1, tf * T))
    masks[0, 11] = np.inf
    masks[0, 5 * tf + 2] = -np.inf
    masks[0, 9 * tf + 40] = np.nan
    masks[0, 20 * tf + 1001] = np.inf
    bands = stx.Bands(sizes, freqs, F, C)
    out = host(bands.scatter_apply(dev(masks[None], device), dev(z[None], device), T, layout=stx.F_MAJOR))[0, 0]
    ref = ob.scatter_apply(sizes, freqs, masks, z.astype(np.complex128), False).astype(np.complex64)[0]
    a, b = out.view(np.float32), ref.view(np.float32)
    assert np.isinf(a).any() and np.isnan(a).any()
    assert np.array_equal(a, b, equal_nan=True)


def test_small_random_table_bit_exact(device, ob):
    from test_oracle_bands import random_table
    sizes, freqs = random_table(5, 33, 9)
    C, F, T, S, batch = 3, 33, 19, 2, 3
    z = rand_spec(14, batch, C, F, T)
    bands = stx.Bands(sizes, freqs, F, C)
    for layout in (stx.F_MAJOR, stx.T_MAJOR):
        zd = z if layout == stx.F_MAJOR else np.ascontiguousarray(z.transpose(0, 1, 3, 2))
        feat = host(bands.gather(dev(zd, device), T, layout=layout))
        masks = synth.uniform(15, (batch, S, bands.total_feat * T))
        out = host(bands.scatter_apply(dev(masks, device), dev(zd, device), T, layout=layout))
        if layout == stx.T_MAJOR:
            out = out.transpose(0, 1, 2, 4, 3)
        for b in range(batch):
            zb = z[b].astype(np.complex128)
            assert np.array_equal(feat[b], ob.gather(sizes, freqs, zb))
            assert np.array_equal(out[b], ob.scatter_apply(sizes, freqs, masks[b], zb).astype(np.complex64))


def two_pair_table():
    """Every bin in at most two (band, position) pairs: overlapping bands, unordered bins, a
    repeated bin, and bins no band covers (the scatter's per-bin record path, not the CSR one)."""
    sizes = [5, 5, 5, 3, 2, 3]
    freqs = [0, 1, 2, 3, 4, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 20, 18, 19, 25, 25, 30, 31, 32]
    return np.array(sizes, np.int32), np.array(freqs, np.int32)


@pytest.mark.parametrize("T,zero_dc", [(1, False), (21, True), (8, False)])
def test_two_pair_table_bit_exact(device, ob, T, zero_dc):
    sizes, freqs = two_pair_table()
    assert np.bincount(freqs, minlength=40).max() == 2
    C, F, S, batch = 3, 40, 3, 2
    z = rand_spec(16, batch, C, F, T)
    bands = stx.Bands(sizes, freqs, F, C)
    masks = synth.uniform(17, (batch, S, bands.total_feat * T))
    for layout in (stx.F_MAJOR, stx.T_MAJOR):
        zd = z if layout == stx.F_MAJOR else np.ascontiguousarray(z.transpose(0, 1, 3, 2))
        feat = host(bands.gather(dev(zd, device), T, layout=layout))
        out = host(bands.scatter_apply(dev(masks, device), dev(zd, device), T, layout=layout, zero_dc=zero_dc))
        if layout == stx.T_MAJOR:
            out = out.transpose(0, 1, 2, 4, 3)
        for b in range(batch):
            zb = z[b].astype(np.complex128)
            assert np.array_equal(feat[b], ob.gather(sizes, freqs, zb))
            ref = ob.scatter_apply(sizes, freqs, masks[b], zb, zero_dc).astype(np.complex64)
            assert np.array_equal(out[b], ref)


@pytest.mark.parametrize("T", [1, 3])
def test_mel_gather_scatter_few_frames(device, ob, mel, T):
    """One or three frames: the T-major gather's workgroups are (pair chunk, frame), 2 chunks
    of the 3,958 pairs per frame here; the scatter's last frame tile is partial."""
    sizes, freqs = mel
    C, F, S, batch = 2, 1025, 2, 3
    z = rand_spec(18, batch, C, F, T)
    bands = stx.Bands(sizes, freqs, F, C)
    masks = synth.uniform(19, (batch, S, bands.total_feat * T))
    zd = np.ascontiguousarray(z.transpose(0, 1, 3, 2))
    feat = host(bands.gather(dev(zd, device), T, layout=stx.T_MAJOR))
    out = host(bands.scatter_apply(dev(masks, device), dev(zd, device), T, layout=stx.T_MAJOR, zero_dc=True))
    out = out.transpose(0, 1, 2, 4, 3)
    for b in range(batch):
        zb = z[b].astype(np.complex128)
        assert np.array_equal(feat[b], ob.gather(sizes, freqs, zb))
        assert np.array_equal(out[b], ob.scatter_apply(sizes, freqs, masks[b], zb, True).astype(np.complex64))


@pytest.mark.parametrize("case", ["mono", "unaligned_out", "wide_frame"])
def test_gather_kernel_paths(device, ob, case):
    """The T-major gather stages a frame in LDS when its C * F complex values fit 64 KB and, at
    C = 2, the output is 16-byte aligned; otherwise it walks the output flat. Both, bit-exact:
    mono (one channel), an output 8 bytes past a 16-byte boundary, and n_fft 8192 stereo
    (2 * 4097 bins, 65.5 KB per frame)."""
    import torch
    n_fft = 8192 if case == "wide_frame" else 2048
    C = 1 if case == "mono" else 2
    F, T, batch = n_fft // 2 + 1, 37, 2
    sizes, freqs = stx.mel_band_map(SR, n_fft, NMELS)
    z = rand_spec(20, batch, C, F, T)
    bands = stx.Bands(sizes, freqs, F, C)
    n = bands.total_feat * T
    zd = dev(np.ascontiguousarray(z.transpose(0, 1, 3, 2)), device)
    if case == "unaligned_out":
        buf = torch.empty(batch * n + 2, dtype=torch.float32, device=device)
        out = buf[2:].view(batch, n)
        assert out.data_ptr() % 16 == 8
        bands.gather(zd, T, layout=stx.T_MAJOR, out=out)
    else:
        out = bands.gather(zd, T, layout=stx.T_MAJOR)
    feat = host(out)
    for b in range(batch):
        assert np.array_equal(feat[b], ob.gather(sizes, freqs, z[b].astype(np.complex128)))


@pytest.mark.parametrize("S", [1, 4])
def test_roformer_spectral_path_c3(device, mel, S):
    # One RoFormer chunk: stereo 352,800 samples, n_fft 2048, hop 441, 60 mel bands; per-band
    # complex masks uniform in [-1, 1]; GPU path in the T-major layout.
    import torch
    sizes, freqs = mel
    orc = oracle_lib.oracle()
    C, L = 2, 352800
    x = synth.normal(2027, (C, L), 0.1)
    fft = stx.FFT(NFFT)
    bands = stx.Bands(sizes, freqs, NFFT // 2 + 1, C)
    spec = stx.torch_stft(fft, dev(x, device), HOP, layout=stx.T_MAJOR)          # [C][T][F]
    T = spec.shape[1]
    feat = bands.gather(spec[None], T)
    masks = dev(synth.uniform(2028, (1, S, bands.total_feat * T)), device)
    y_spec = bands.scatter_apply(masks, spec[None], T)[0]                         # [S][C][T][F]
    y = stx.torch_istft(fft, y_spec.reshape(S * C, T, NFFT // 2 + 1), HOP, layout=stx.T_MAJOR)
    y = host(y).reshape(S, C, -1)
    # Oracle: double STFT, band masks, double iSTFT.
    z = np.stack([orc.torch_stft(x[c], NFFT, HOP) for c in range(C)])             # [C][F][T]
    feat_ref = oracle_lib.bands().gather(sizes, freqs, z)
    assert snr_db(host(feat)[0], feat_ref) >= 110.0
    ys = oracle_lib.bands().scatter_apply(sizes, freqs, host(masks)[0], z)        # [S][C][F][T]
    for s in range(S):
        for c in range(C):
            yref = orc.torch_istft(ys[s, c], NFFT, HOP)
            assert snr_db(y[s, c], yref) >= 110.0
    del torch


def test_all_ones_masks_reconstruct_input(device, mel):
    # An all-ones mask in every band averages to 1 on every bin, so the path is STFT -> iSTFT.
    sizes, freqs = mel
    C, L = 2, 44100 * 2
    x = synth.normal(31, (C, L), 0.1)
    fft = stx.FFT(NFFT)
    bands = stx.Bands(sizes, freqs, NFFT // 2 + 1, C)
    spec = stx.torch_stft(fft, dev(x, device), HOP, layout=stx.T_MAJOR)
    T = spec.shape[1]
    import torch
    ones = torch.ones((1, 1, bands.total_feat * T), dtype=torch.float32, device=device)
    ones[..., 1::2] = 0.0                                                          # 1 + 0i
    out = bands.scatter_apply(ones, spec[None], T)[0, 0]
    y = host(stx.torch_istft(fft, out, HOP, layout=stx.T_MAJOR))
    n = (T - 1) * HOP
    assert snr_db(y, x[:, :n]) >= 110.0


def test_band_table_errors(device):
    with pytest.raises(stx.StxError) as e:
        stx.Bands(np.array([2, 2], np.int32), np.array([0, 1, 2], np.int32), 8, 2)
    assert e.value.status == stx.STATUS_RUNTIME_ERROR


# ------------------------------------------------- band-split RMSNorm and mask-head GLU
def band_blocks(sizes, C, T):
    """(offset, dim_in) of each band's [T][dim_in] block in a [total_feat * T] buffer."""
    out, off = [], 0
    for s in sizes:
        din = int(s) * C * 2
        out.append((off, din))
        off += din * T
    return out


@pytest.mark.parametrize("kind,T,batch", [("mel", 801, 2), ("bs", 801, 1), ("mel", 17, 3)])
def test_band_rms_norm(device, mel, kind, T, batch):
    """src/roformer.cpp:169-175: rms(view_b, band.b.norm) for every band, against the oracle's
    RMSNorm (double, rounded once) on each band's rows."""
    import torch
    ops = oracle_lib.ops()
    sizes, freqs = mel if kind == "mel" else (np.array(BS_FPB, np.int32), np.arange(1025, dtype=np.int32))
    C = 2
    bands = stx.Bands(sizes, freqs, 1025, C)
    feat = synth.normal(21, (batch, bands.total_feat * T), 0.7)
    gam = [synth.normal(100 + b, (int(s) * C * 2,), 1.0) for b, s in enumerate(sizes)]
    gd = [dev(g, device) for g in gam]
    y = host(bands.rms_norm(dev(feat, device), T, gd, eps=1e-24))
    for bi in range(batch):
        for (off, din), g in zip(band_blocks(sizes, C, T), gam):
            x = feat[bi, off:off + din * T].reshape(T, din)
            want = ops.norm(x, 1e-24, rms=True, w=g)
            got = y[bi, off:off + din * T].reshape(T, din)
            assert rel_err(got, want) <= 1e-6
    # In place, and equal to stx_rms_norm_mul on one band's view.
    fd = dev(feat, device)
    bands.rms_norm(fd, T, gd, out=fd)
    assert np.array_equal(host(fd), y)
    off, din = band_blocks(sizes, C, T)[5]
    view = dev(feat[0, off:off + din * T].reshape(T, din), device)
    one = host(stx.rms_norm(view, 1e-24, gamma=gd[5]))
    assert rel_err(y[0, off:off + din * T].reshape(T, din), one) <= 1e-6


@pytest.mark.parametrize("C,misalign", [(1, False), (2, True), (3, False)])
def test_band_rms_norm_float2_kernel(device, mel, C, misalign):
    """The float2 kernel, taken for an odd channel count or a buffer that is not 16-byte aligned
    (the float4 kernel needs neither): the same oracle bound."""
    import torch
    ops = oracle_lib.ops()
    sizes, freqs = mel
    T = 37
    bands = stx.Bands(sizes, freqs, 1025, C)
    feat = synth.normal(31 + C, (1, bands.total_feat * T), 0.7)
    gam = [synth.normal(200 + b, (int(s) * C * 2,), 1.0) for b, s in enumerate(sizes)]
    if misalign:       # gamma of band 3 one float past a 16-byte boundary
        g3 = torch.zeros(gam[3].size + 1, dtype=torch.float32, device=device)
        g3[1:] = dev(gam[3], device)
        gd = [dev(g, device) for g in gam]
        gd[3] = g3[1:]
        assert gd[3].data_ptr() % 16 != 0
    else:
        gd = [dev(g, device) for g in gam]
    y = host(bands.rms_norm(dev(feat, device), T, gd, eps=1e-24))
    for (off, din), g in zip(band_blocks(sizes, C, T), gam):
        x = feat[0, off:off + din * T].reshape(T, din)
        assert rel_err(y[0, off:off + din * T].reshape(T, din), ops.norm(x, 1e-24, rms=True, w=g)) <= 1e-6


@pytest.mark.parametrize("kind,S,T", [("mel", 4, 801), ("bs", 2, 801), ("mel", 9, 33)])
def test_band_mask_glu(device, mel, kind, S, T):
    """src/roformer.cpp:199-204: GLU on dim 0 of every (stem, band) head into the mask layout
    the scatter reads; bit-identical to stx_glu per band, within 1e-6 of the oracle's GLU."""
    ops = oracle_lib.ops()
    sizes, freqs = mel if kind == "mel" else (np.array(BS_FPB, np.int32), np.arange(1025, dtype=np.int32))
    C = 2
    bands = stx.Bands(sizes, freqs, 1025, C)
    heads_h = [synth.normal(1000 * s + b, (T, 2 * int(z) * C * 2), 2.0) for s in range(S) for b, z in enumerate(sizes)]
    heads = [dev(h, device) for h in heads_h]
    m = host(bands.mask_glu(heads, S, T))
    blocks = band_blocks(sizes, C, T)
    for s in range(S):
        for b, (off, din) in enumerate(blocks):
            h = heads_h[s * len(sizes) + b]
            got = m[s, off:off + din * T].reshape(T, din)
            want = ops.glu(h, 0)
            assert rel_err(got, want) <= 1e-6
            if b % 17 == 0:
                assert np.array_equal(got, host(stx.glu(heads[s * len(sizes) + b], 0)))


def test_band_mask_glu_many_stems(device):
    """More (stem, band) heads than one launch carries: 40 stems of 60 bands."""
    sizes = np.array([1, 2, 3] * 20, np.int32)
    freqs = np.arange(int(sizes.sum()), dtype=np.int32) % 100
    C, T, S = 2, 5, 40
    bands = stx.Bands(sizes, freqs, 100, C)
    heads_h = [synth.normal(7 + i, (T, 2 * int(z) * C * 2), 1.0) for i, z in enumerate(np.tile(sizes, S))]
    m = host(bands.mask_glu([dev(h, device) for h in heads_h], S, T))
    ops = oracle_lib.ops()
    blocks = band_blocks(sizes, C, T)
    for s in range(S):
        for b, (off, din) in enumerate(blocks):
            want = ops.glu(heads_h[s * 60 + b], 0)
            assert rel_err(m[s, off:off + din * T].reshape(T, din), want) <= 1e-6
