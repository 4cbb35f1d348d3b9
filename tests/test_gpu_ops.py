"""GPU parity of the ggml ops (ops.hip) against the oracle at the shapes the reference runs.

Bar: rel_err <= 1e-6 (max |a - b| / max(|b|, 1e-6 rms(b))) for the normalisations, softmax,
GELU, GLU and RoPE, which the oracle evaluates in double and rounds once; bit-exact for ADD,
MUL and the LayerScale + residual x + h*s, which round after every operation.

Shapes: HTDemucs GroupNorm/GELU/GLU/LayerScale at [T, 1, C] for (C, T) in {(48, 85995),
(96, 21499), (192, 5375), (384, 1344)}; RoFormer RMSNorm at 48,060 rows x 384 and the band-split
widths, softmax at one 256 MiB score group [801, 801, 8, 13] and [60, 60, 8, 801] and the HTDemucs
scores [Nk, Nq, 8] for Nk, Nq in {1344, 2688}, the FF bias +
GELU at [1536, 801, 60], RoPE at [64, 8, 801, 60] and [64, 8, 60, 801] (ggml order, ne0 first;
numpy shapes below are reversed).
"""
import numpy as np
import pytest

import oracle_lib
import stx
from metrics import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-6


@pytest.fixture(scope="module")
def ops():
    return oracle_lib.ops()


def randn(device, shape, seed, sigma=1.0, mean=0.0):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32) * sigma + mean


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


HTDEMUCS_CT = [(48, 85995), (96, 21499), (192, 5375), (384, 1344), (6, 85995)]


# ------------------------------------------------------------------- GROUP_NORM
@pytest.mark.parametrize("C,T", HTDEMUCS_CT + [(47, 85993)])    # last: odd-sized group (no float4 path)
@pytest.mark.parametrize("gelu", [False, True])
def test_group_norm_rows_h1(device, ops, C, T, gelu):
    """group_norm_rows with H == 1 (src/htdemucs.cpp:117-119,127): G = 1 over [T, 1, C], * w[C] + b[C]."""
    x = randn(device, (C, 1, T), C + T, 1.7, 0.3)
    w = randn(device, (C, 1, 1), 1, 1.0)
    b = randn(device, (C, 1, 1), 2, 1.0)
    y = host(stx.group_norm(x, 1, 1e-5, w, b, gelu=gelu))
    want = ops.group_norm(host(x), 1, 1e-5, host(w), host(b), gelu=gelu)
    assert rel_err(y, want) <= TOL


@pytest.mark.parametrize("W,C,H", [(336, 48, 8), (85, 96, 32), (1000, 6, 3)])
def test_group_norm_rows_h_groups(device, ops, W, C, H):
    """H > 1 (src/htdemucs.cpp:120-126): [W, C, H] with H groups, affine over C = ne1 (general broadcast)."""
    x = randn(device, (H, C, W), W + C, 1.0, -0.2)
    w = randn(device, (1, C, 1), 3, 1.0)
    b = randn(device, (1, C, 1), 4, 1.0)
    y = host(stx.group_norm(x, H, 1e-5, w, b))
    want = ops.group_norm(host(x), H, 1e-5, host(w), host(b))
    assert rel_err(y, want) <= TOL


def test_group_norm_norm_out(device, ops):
    """norm_out (src/htdemucs.cpp:223-227): G = 1 over [D, N], weight/bias over D (ne0)."""
    D, N = 384, 2689
    x = randn(device, (N, D), 5, 2.0, 1.0)
    w, b = randn(device, (D,), 6), randn(device, (D,), 7)
    y = host(stx.group_norm(x, 1, 1e-5, w, b))
    assert rel_err(y, ops.group_norm(host(x), 1, 1e-5, host(w), host(b))) <= TOL


def test_group_norm_ragged_groups_and_batches(device, ops):
    # ne2 = 7 channels in 3 groups (3, 3, 1), ne3 = 2 slices, plane of 13 floats (no float4 path).
    x = randn(device, (2, 7, 1, 13), 8, 3.0, 5.0)
    y = host(stx.group_norm(x, 3))
    assert rel_err(y, ops.group_norm(host(x), 3)) <= TOL


def test_group_norm_in_place_and_deterministic(device, ops):
    C, T = 48, 85995
    x = randn(device, (C, 1, T), 9, 1.0)
    xh = host(x)
    a = host(stx.group_norm(x, 1))
    b = host(stx.group_norm(x, 1))
    assert np.array_equal(a, b)
    stx.group_norm(x, 1, out=x)
    assert np.array_equal(host(x), a)
    assert rel_err(a, ops.group_norm(xh, 1)) <= TOL


@pytest.mark.parametrize("gelu", [False, True])
def test_group_norm_shapes_share_a_workspace(device, ops, gelu):
    """Large groups, many groups and batched groups: one workspace, filled with garbage first,
    serves all of them in turn, twice (no initialisation needed: the single-pass kernel's
    records are keyed by the dispatch, and the two-pass areas are written before they are read)."""
    import torch
    ws = torch.full((1 << 17,), -7.25, device=device)
    shapes = [((96, 1, 85995), 1), ((1000, 1, 8192), 1000), ((48, 1, 85995), 1), ((8, 3, 1, 999), 4)]
    for rep in range(2):
        for shape, G in shapes:
            x = randn(device, shape, shape[0] + rep, 1.5, 0.5)
            C = shape[-3]
            w, b = randn(device, (C, 1, 1), 1), randn(device, (C, 1, 1), 2)
            assert stx.group_norm_workspace_size(x, G) <= ws.numel() * 4
            y = host(stx.group_norm(x, G, 1e-5, w, b, gelu=gelu, workspace=ws))
            assert rel_err(y, ops.group_norm(host(x), G, 1e-5, host(w), host(b), gelu=gelu)) <= TOL


def test_group_norm_graph_replays(device, ops):
    """Replays of one captured call on new data each time: the single-pass kernel's records are
    keyed by the dispatch, so a replay must wait for its own records, not take the last one's."""
    import torch
    C, T = 96, 21499
    x = randn(device, (C, 1, T), 40)
    w, b = randn(device, (C, 1, 1), 41), randn(device, (C, 1, 1), 42)
    y = torch.empty_like(x)
    ws = stx.workspace(stx.group_norm_workspace_size(x, 1), device)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        stx.group_norm(x, 1, 1e-5, w, b, gelu=True, out=y, workspace=ws, stream=s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            stx.group_norm(x, 1, 1e-5, w, b, gelu=True, out=y, workspace=ws, stream=s)
    torch.cuda.synchronize()
    for rep in range(4):
        xn = randn(device, (C, 1, T), 50 + rep, 1.0 + rep, 0.1 * rep)
        x.copy_(xn)
        torch.cuda.synchronize()
        g.replay()
        want = ops.group_norm(host(xn), 1, 1e-5, host(w), host(b), gelu=True)
        assert rel_err(host(y), want) <= TOL


@pytest.mark.parametrize("C,T", [(96, 21499), (384, 1344)])
def test_group_norm_without_grid_sync(device, ops, C, T, monkeypatch):
    """STX_NO_GRID_SYNC=1 sends shapes that take the single pass to the two-kernel path: both
    paths give the oracle's result."""
    x = randn(device, (C, 1, T), 60 + C, 1.3, -0.4)
    w, b = randn(device, (C, 1, 1), 61), randn(device, (C, 1, 1), 62)
    want = ops.group_norm(host(x), 1, 1e-5, host(w), host(b), gelu=True)
    y1 = host(stx.group_norm(x, 1, 1e-5, w, b, gelu=True))
    monkeypatch.setenv("STX_NO_GRID_SYNC", "1")
    y2 = host(stx.group_norm(x, 1, 1e-5, w, b, gelu=True))
    assert rel_err(y1, want) <= TOL and rel_err(y2, want) <= TOL


GN_PATH_SHAPES = [((96, 1, 21499), 1), ((384, 1, 1344), 1), ((8, 1, 3000), 4), ((64, 1, 100), 1),
                  ((47, 1, 21497), 1), ((47, 1, 85993), 1), ((2, 6, 1, 700), 3)]


@pytest.mark.parametrize("shape,G", GN_PATH_SHAPES)
@pytest.mark.parametrize("gelu", [False, True])
def test_group_norm_paths_same_bits(device, ops, shape, G, gelu, monkeypatch):
    """Every path gives the same bits: the single pass; two passes (STX_NO_GRID_SYNC=1); in
    place (two passes, since a single-pass block may have to re-read x); and the single pass
    with every wait given up at its first look (STX_GRID_SYNC_SPIN_LIMIT=0), where each block
    that gives up computes its group's totals from x itself. Only the forced run counts
    fallbacks in its workspace. Shapes: per-wave channel parameters (planes >= 256), per-element
    ones (plane 100), unaligned group spans (no float4 loads) below and above 2^21 floats
    (groups of more than 512 chunks of 4096 floats take two passes in every run), several
    groups per launch and a batch (ne3 = 2) of ragged groups."""
    import torch
    x = randn(device, shape, sum(shape) + G, 1.3, 0.7)
    C = shape[-3]
    w, b = randn(device, (C, 1, 1), 70), randn(device, (C, 1, 1), 71)
    ws = stx.workspace(stx.group_norm_workspace_size(x, G), device)
    y1 = host(stx.group_norm(x, G, 1e-5, w, b, gelu=gelu, workspace=ws))
    assert stx.grid_sync_fallbacks(ws) == 0
    assert rel_err(y1, ops.group_norm(host(x), G, 1e-5, host(w), host(b), gelu=gelu)) <= TOL
    monkeypatch.setenv("STX_NO_GRID_SYNC", "1")
    y2 = host(stx.group_norm(x, G, 1e-5, w, b, gelu=gelu))
    monkeypatch.delenv("STX_NO_GRID_SYNC")
    xc = x.clone()
    stx.group_norm(xc, G, 1e-5, w, b, gelu=gelu, out=xc)
    y3 = host(xc)
    ws0 = stx.workspace(stx.group_norm_workspace_size(x, G), device)
    monkeypatch.setenv("STX_GRID_SYNC_SPIN_LIMIT", "0")
    y4 = host(stx.group_norm(x, G, 1e-5, w, b, gelu=gelu, workspace=ws0))
    monkeypatch.delenv("STX_GRID_SYNC_SPIN_LIMIT")
    forced = stx.grid_sync_fallbacks(ws0)
    assert np.array_equal(y1, y2) and np.array_equal(y1, y3) and np.array_equal(y1, y4)
    ne = list(shape[::-1]) + [1] * (4 - len(shape))
    cpg = -(-ne[2] // G)
    span, groups_total = cpg * ne[0] * ne[1], -(-ne[2] // cpg) * ne[3]
    vec = 1 if span <= 512 * 2048 else 2 if span <= 512 * 4096 else 4
    chunks = -(-span // (2048 * vec))
    if vec < 4 and groups_total <= 8 and chunks <= 512 and chunks > 1:   # a single pass whose blocks wait
        assert forced > 0


def test_group_norm_errors(device):
    import torch
    x = randn(device, (4, 1, 100), 10)
    ws = stx.workspace(8, device)
    with pytest.raises(stx.StxError) as e:
        stx.group_norm(x, 1, workspace=ws)                  # one 100-float group needs 16 bytes
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    with pytest.raises(stx.StxError) as e:
        stx.group_norm(x, 0)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    with pytest.raises(stx.StxError) as e:
        stx.group_norm(x, 1, weight=randn(device, (3, 1, 1), 1))   # 3 does not repeat into 4
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    with pytest.raises(stx.StxError) as e:
        stx.group_norm(x[:, :, ::2], 1)                        # not contiguous
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    empty = torch.empty((0, 1, 5), device=device)
    stx.group_norm(empty, 1)


# ------------------------------------------------------------------ NORM / RMS_NORM
@pytest.mark.parametrize("rows,n", [(48060, 384), (801, 24), (801, 520), (801, 132), (37, 1), (5, 2048), (9, 3001)])
def test_rms_norm_mul(device, ops, rows, n):
    """Graph::rms (src/roformer.cpp:96-98) with eps 1e-24 (:34)."""
    x = randn(device, (rows, n), rows + n, 1.3, 0.1)
    g = randn(device, (n,), n)
    y = host(stx.rms_norm(x, 1e-24, gamma=g))
    assert rel_err(y, ops.norm(host(x), 1e-24, rms=True, w=host(g))) <= TOL
    y0 = host(stx.rms_norm(x, 1e-24))
    assert rel_err(y0, ops.norm(host(x), 1e-24, rms=True)) <= TOL


def test_rms_norm_zero_rows(device):
    import torch
    x = torch.zeros((3, 384), device=device)
    assert np.all(host(stx.rms_norm(x, 1e-24)) == 0.0)


@pytest.mark.parametrize("rows,n", [(2688, 384), (100, 512), (7, 5000), (33, 96)])
def test_norm_and_layer_norm(device, ops, rows, n):
    """ggml_norm (src/htdemucs.cpp:215) and layer_norm = norm * w + b (:213-215), eps 1e-5."""
    x = randn(device, (rows, n), rows * n, 2.0, 3.0)
    w, b = randn(device, (n,), 11), randn(device, (n,), 12)
    assert rel_err(host(stx.norm(x, 1e-5)), ops.norm(host(x), 1e-5)) <= TOL
    y = host(stx.norm(x, 1e-5, weight=w, bias=b))
    assert rel_err(y, ops.norm(host(x), 1e-5, w=host(w), b=host(b))) <= TOL


def test_norm_strided_rows_in_place(device, ops):
    big = randn(device, (64, 2, 300), 13)
    v = big[:, 0, :]                                         # rows 2400 bytes apart
    want = ops.norm(host(v), 1e-5)
    stx.norm(v, 1e-5, out=v)
    assert rel_err(host(v), want) <= TOL


def test_row_ops_output_misaligned_with_input(device, ops):
    """Rows whose output starts at a different offset modulo 16 bytes than the input take the
    scalar-load kernels; rows with any head/tail split take the vector-load ones (801 floats)."""
    import torch
    rows, n = 300, 801
    x = randn(device, (rows, n), 31, 2.0)
    buf = torch.empty(rows * n + 1, device=device)
    out = buf[1:].view(rows, n)                      # 4 bytes off the input's alignment
    xh = host(x)
    assert rel_err(host(stx.rms_norm(x, 1e-24, out=out)), ops.norm(xh, 1e-24, rms=True)) <= TOL
    assert rel_err(host(stx.soft_max_ext(x, 0.125, out=out)), ops.soft_max(xh, 0.125)) <= TOL
    assert rel_err(host(stx.norm(x, 1e-5, out=out)), ops.norm(xh, 1e-5)) <= TOL


# ------------------------------------------------------------------------ SOFT_MAX
@pytest.mark.parametrize("shape,sigma", [((13, 8, 801, 801), 8.0), ((801, 8, 60, 60), 8.0), ((4, 8, 801, 801), 60.0),
                                         ((3, 1000), 1.0), ((2, 2048), 4.0), ((17, 1), 1.0)])
def test_soft_max_ext(device, ops, shape, sigma):
    """ggml_soft_max_ext(kq, NULL, 1/sqrt(64), 0) (src/roformer.cpp:127)."""
    x = randn(device, shape, int(np.prod(shape)) % 1000, sigma)
    y = stx.soft_max_ext(x, 0.125)
    n0 = shape[-1]
    want = ops.soft_max(host(x).reshape(-1, n0), 0.125)
    assert rel_err(host(y).reshape(-1, n0), want) <= TOL


def test_soft_max_negative_scale_and_errors(device, ops):
    x = randn(device, (50, 333), 14, 3.0)
    assert rel_err(host(stx.soft_max_ext(x, -0.7)), ops.soft_max(host(x), -0.7)) <= TOL
    with pytest.raises(stx.StxError) as e:
        stx.soft_max_ext(x, 0.125, mask=x)
    assert e.value.status == stx.STATUS_UNSUPPORTED
    with pytest.raises(stx.StxError) as e:
        stx.soft_max_ext(x, 0.125, max_bias=8.0)
    assert e.value.status == stx.STATUS_UNSUPPORTED


HTDEMUCS_KQ = [(2688, 2688), (1344, 2688), (2688, 1344), (1344, 1344)]


@pytest.mark.parametrize("nk,nq", HTDEMUCS_KQ)
@pytest.mark.parametrize("hd", [48, 64])
def test_soft_max_htdemucs(device, ops, nk, nq, hd):
    """ggml_soft_max_ext(kq, NULL, 1/sqrt((float)hd), 0) over kq [Nk, Nq, 8] (src/htdemucs.cpp:236-238):
    Nk and Nq are the 8 x 336 = 2,688 frequency tokens (:354-358) or the 1,344 time tokens, hd =
    D / 8 with D = 384 or 512 (the widened bottom). Rows of 2,688 take one block per row."""
    x = randn(device, (8, nq, nk), nk + nq + hd, 6.0)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    y = stx.soft_max_ext(x, scale)
    want = ops.soft_max(host(x).reshape(-1, nk), scale)
    assert rel_err(host(y).reshape(-1, nk), want) <= TOL


@pytest.mark.parametrize("n", [2049, 2688, 3072, 3073, 4096, 5000, 6144, 8192, 8193, 20000])
def test_soft_max_long_rows(device, ops, n):
    """Rows longer than 2048: aligned rows, rows starting 4 bytes past a 16-byte boundary (a
    head of 3 floats), an output misaligned with the input (the three-pass kernel) and the
    call in place."""
    import torch
    rows = 37
    buf = randn(device, (rows * n + 8,), n, 5.0)
    for off in (0, 1):
        x = buf[off:off + rows * n].view(rows, n)
        xh = host(x)
        want = ops.soft_max(xh, 0.2)
        assert rel_err(host(stx.soft_max_ext(x, 0.2)), want) <= TOL
        out = torch.empty(rows * n + 1, device=device)[1 - off:1 - off + rows * n].view(rows, n)
        assert rel_err(host(stx.soft_max_ext(x, 0.2, out=out)), want) <= TOL
        xc = x.clone()
        assert rel_err(host(stx.soft_max_ext(xc, 0.2, out=xc)), want) <= TOL
    neg = buf[:rows * n].view(rows, n)
    assert rel_err(host(stx.soft_max_ext(neg, -0.3)), ops.soft_max(host(neg), -0.3)) <= TOL


# ---------------------------------------------------------------------------- GELU
def test_gelu_ff_bias(device, ops):
    """FF: ggml_gelu_erf(linear + bias) at [1536, 801, 60] (src/roformer.cpp:147)."""
    h = randn(device, (60, 801, 1536), 15, 1.5)
    bias = randn(device, (1536,), 16, 0.5)
    y = host(stx.gelu_erf(h, bias=bias))
    hh, bh = host(h), host(bias)
    assert rel_err(y, ops.binary("add_gelu", hh, bh)) <= TOL
    y0 = host(stx.gelu_erf(h))
    assert rel_err(y0, ops.gelu(hh)) <= TOL


def test_gelu_tails_and_specials(device, ops):
    import torch
    xs = np.concatenate([np.linspace(-14, 14, 200001, dtype=np.float32),
                         np.array([0.0, -0.0, 1e-30, -1e-30, 3e38, -3e38, np.inf, -np.inf], np.float32)])
    x = torch.from_numpy(xs).to(device)
    y = host(stx.gelu_erf(x))
    want = ops.gelu(xs)
    assert rel_err(y[:200001], want[:200001]) <= TOL
    # Element by element, relative to each value (the negative tail included, down to
    # gelu(-14) ~ 1e-43 where float runs out): within 16 * 2^-24 (< 1e-6) of the oracle's
    # double-precision value rounded to float.
    yv, wv = y[:200001].astype(np.float64), want[:200001].astype(np.float64)
    m = np.abs(wv) > 1e-36
    assert np.max(np.abs(yv[m] - wv[m]) / np.abs(wv[m])) <= 16 * 2.0**-24
    sp, wsp = y[200001:], want[200001:]
    # 0, -0, +-1e-30, +-3e38 to the closed form; gelu(inf) = inf, gelu(-inf) = -inf * 0 = NaN.
    assert np.array_equal(sp[:6], wsp[:6])
    assert sp[6] == np.inf and wsp[6] == np.inf
    assert np.isnan(sp[7]) and np.isnan(wsp[7])


# ----------------------------------------------------------------------------- GLU
@pytest.mark.parametrize("C,T", HTDEMUCS_CT[:4])
def test_glu_channels(device, ops, C, T):
    """glu over ne2 of [T, 1, 2C] (src/htdemucs.cpp:105-110)."""
    x = randn(device, (2 * C, 1, T), C, 2.0)
    assert rel_err(host(stx.glu(x, 2)), ops.glu(host(x), 2)) <= TOL


@pytest.mark.parametrize("din", [24, 520, 132])
def test_glu_mask_head(device, ops, din):
    """Mask estimator GLU on dim 0 of [2 dim_in, T] (src/roformer.cpp:199-202)."""
    x = randn(device, (801, 2 * din), din, 3.0)
    assert rel_err(host(stx.glu(x, 0)), ops.glu(host(x), 0)) <= TOL


# ------------------------------------------------------------------ ADD / MUL (exact)
@pytest.mark.parametrize("C,T", HTDEMUCS_CT)
def test_layer_scale_residual_bit_exact(device, ops, C, T):
    """x + h * scale[C] (src/htdemucs.cpp:139)."""
    x, h = randn(device, (C, 1, T), 20), randn(device, (C, 1, T), 21)
    s = randn(device, (C, 1, 1), 22, 1e-2)
    y = host(stx.mul_add(x, h, s))
    assert np.array_equal(y, ops.binary("mul_add", host(x), host(h), host(s)))


@pytest.mark.parametrize("C,T", HTDEMUCS_CT)
def test_glu_layer_scale_residual_fused_bit_exact(device, C, T):
    """x + glu(h) * scale (src/htdemucs.cpp:137-139) in one kernel is bit-identical to the
    GLU and the LayerScale + residual run separately (each checked against the oracle above)."""
    h = randn(device, (2 * C, 1, T), C, 2.0)
    x, s = randn(device, (C, 1, T), C + 1), randn(device, (C, 1, 1), C + 2, 0.1)
    fused = host(stx.glu_mul_add(x, h, 2, s))
    sep = host(stx.mul_add(x, stx.glu(h, 2), s))
    assert np.array_equal(fused, sep)


def test_glu_layer_scale_residual_dim0_and_errors(device):
    h = randn(device, (801, 2 * 132), 5, 2.0)
    x, s = randn(device, (801, 132), 6), randn(device, (132,), 7)
    assert np.array_equal(host(stx.glu_mul_add(x, h, 0, s)), host(stx.mul_add(x, stx.glu(h, 0), s)))
    with pytest.raises(stx.StxError) as e:
        stx.glu_mul_add(x, randn(device, (801, 263), 1), 0, s)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT


@pytest.mark.parametrize("shape,bshape", [((60, 801, 1536), (1536,)), ((48, 1, 85995), (48, 1, 1)),
                                          ((801, 60, 8, 64), (801, 60, 8, 1)), ((7, 5, 3), (7, 5, 3)),
                                          ((4, 6, 8), (1, 6, 1)), ((3, 1021), (1, 1021))])
def test_add_mul_broadcast_bit_exact(device, ops, shape, bshape):
    a, b = randn(device, shape, 23), randn(device, bshape, 24)
    ah, bh = host(a), host(b)
    assert np.array_equal(host(stx.add(a, b)), ops.binary("add", ah, bh))
    assert np.array_equal(host(stx.mul(a, b)), ops.binary("mul", ah, bh))


def test_binary_strided_views(device, ops):
    big = randn(device, (40, 3, 257), 25)
    a = big[:, 1, :]                                         # non-contiguous rows
    b = randn(device, (257,), 26)
    assert np.array_equal(host(stx.add(a, b)), ops.binary("add", host(a), host(b)))
    with pytest.raises(stx.StxError) as e:
        stx.add(a, randn(device, (256,), 1))
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT


# ---------------------------------------------------------------------------- ROPE
@pytest.mark.parametrize("shape", [(60, 801, 8, 64), (801, 60, 8, 64)])
def test_rope_roformer(device, ops, shape):
    """ggml_rope_ext(t, pos, NULL, 64, 0, 0, 1e4, 1, 0, 1, 0, 0) (src/roformer.cpp:109-110)
    over [dh, H, N, batch] with positions 0..N-1 (:242-247)."""
    import torch
    x = randn(device, shape, shape[1])
    N = shape[1]
    pos = torch.arange(N, dtype=torch.int32, device=device)
    y = host(stx.rope_ext(x, pos, 64))
    assert rel_err(y, ops.rope(host(x), np.arange(N, dtype=np.int32), 64)) <= TOL


def test_rope_neox_partial_dims_in_place(device, ops):
    import torch
    x = randn(device, (3, 20, 5, 48), 27)
    posh = (np.arange(20, dtype=np.int32) * 7) % 13
    pos = torch.from_numpy(posh).to(device)
    xh = host(x)
    want2 = ops.rope(xh, posh, 32, mode=2, freq_base=500.0, freq_scale=0.5, attn_factor=1.5)
    y2 = host(stx.rope_ext(x, pos, 32, mode=2, freq_base=500.0, freq_scale=0.5, attn_factor=1.5))
    assert rel_err(y2, want2) <= TOL
    want0 = ops.rope(xh, posh, 32)
    stx.rope_ext(x, pos, 32, out=x)
    assert rel_err(host(x), want0) <= TOL


def test_rope_mode0_rows_not_multiple_of_4(device, ops):
    """ne0 = 50 (not a multiple of 4 floats) takes the pair-per-thread kernel, 64 the float4 one;
    both against the oracle."""
    import torch
    for ne0, nd in [(50, 46), (64, 64), (52, 40)]:
        x = randn(device, (2, 33, 4, ne0), ne0)
        posh = np.arange(33, dtype=np.int32) * 5
        y = host(stx.rope_ext(x, torch.from_numpy(posh).to(device), nd))
        assert rel_err(y, ops.rope(host(x), posh, nd)) <= TOL


def test_rope_errors(device):
    import torch
    x = randn(device, (1, 4, 2, 64), 28)
    pos = torch.arange(4, dtype=torch.int32, device=device)
    with pytest.raises(stx.StxError) as e:
        stx.rope_ext(x, pos, 64, ext_factor=1.0)
    assert e.value.status == stx.STATUS_UNSUPPORTED
    with pytest.raises(stx.StxError) as e:
        stx.rope_ext(x, pos, 64, mode=8)
    assert e.value.status == stx.STATUS_UNSUPPORTED
    with pytest.raises(stx.StxError) as e:
        stx.rope_ext(x, pos, 66)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
