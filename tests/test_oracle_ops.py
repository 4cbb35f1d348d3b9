"""CPU checks that pin the ggml op oracle (oracle/ops_oracle.c).

ggml's sources are not part of the reference tree, so no reference test or golden vector
covers these ops. The oracle is pinned against torch's float64 implementations (an
independent library, not the reference), against a complex-number restatement of RoPE, and
against invariants that a dropped term, a wrong sign or a transposed index would break.
ADD/MUL/MUL_ADD are checked bit for bit against numpy's float32 arithmetic.
"""
import numpy as np
import pytest

import oracle_lib
import synth
from metrics import rel_err

TOL = 1e-6


@pytest.fixture(scope="module")
def ops():
    return oracle_lib.ops()


def t64(a):
    import torch
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


# ------------------------------------------------------------------- GROUP_NORM
@pytest.mark.parametrize("N,C,H,W,G", [(1, 48, 1, 997, 1), (2, 12, 3, 50, 4), (1, 6, 5, 7, 6), (3, 8, 1, 33, 2)])
def test_group_norm_vs_torch(ops, N, C, H, W, G):
    import torch.nn.functional as F
    x = synth.normal(C * W + G, (N, C, H, W), 2.0) + 0.75
    w = synth.normal(C, (C,), 1.0)
    b = synth.normal(C + 1, (C,), 1.0)
    got = ops.group_norm(x, G, 1e-5, w.reshape(C, 1, 1), b.reshape(C, 1, 1))
    want = F.group_norm(t64(x), G, t64(w), t64(b), eps=1e-5).numpy()
    assert rel_err(got, want) <= TOL
    got_g = ops.group_norm(x, G, 1e-5, w.reshape(C, 1, 1), b.reshape(C, 1, 1), gelu=True)
    want_g = F.gelu(F.group_norm(t64(x), G, t64(w), t64(b), eps=1e-5)).numpy()
    assert rel_err(got_g, want_g) <= TOL


def test_group_norm_uneven_groups(ops):
    # ne2 = 5 channels in 2 groups: ceil(5/2) = 3 channels, then 2 (ggml's split).
    x = synth.normal(3, (2, 5, 4, 9), 1.0) * np.arange(1, 6, dtype=np.float32)[None, :, None, None]
    got = ops.group_norm(x, 2)
    for n in range(2):
        for c0, c1 in [(0, 3), (3, 5)]:
            g = x[n, c0:c1].astype(np.float64)
            want = (g - g.mean()) / np.sqrt(g.var() + 1e-5)
            assert rel_err(got[n, c0:c1], want) <= TOL


def test_group_norm_invariants(ops):
    x = synth.normal(5, (1, 16, 1, 4000), 3.0) + 100.0          # large mean: no cancellation
    y = ops.group_norm(x, 4).astype(np.float64)
    for g in range(4):
        blk = y[0, 4 * g:4 * g + 4]
        var = x[0, 4 * g:4 * g + 4].astype(np.float64).var()
        assert abs(blk.mean()) < 1e-6
        assert abs(blk.var() - var / (var + 1e-5)) < 1e-6


def test_group_norm_affine_broadcast_ne0(ops):
    # norm_out of src/htdemucs.cpp:223-227: G = 1 over [D, N] with weight/bias over D (ne0).
    D, N = 64, 37
    x = synth.normal(8, (N, D), 1.0)
    w, b = synth.normal(9, (D,), 1.0), synth.normal(10, (D,), 1.0)
    got = ops.group_norm(x, 1, 1e-5, w, b)
    g = x.astype(np.float64)
    want = (g - g.mean()) / np.sqrt(g.var() + 1e-5) * w + b
    assert rel_err(got, want) <= TOL


# ------------------------------------------------------------------ NORM / RMS_NORM
@pytest.mark.parametrize("n", [1, 24, 384, 520, 3000])
def test_norm_vs_torch(ops, n):
    import torch.nn.functional as F
    x = synth.normal(n, (7, n), 1.5) + 0.5
    w, b = synth.normal(n + 1, (n,), 1.0), synth.normal(n + 2, (n,), 1.0)
    assert rel_err(ops.norm(x, 1e-5), F.layer_norm(t64(x), (n,), eps=1e-5).numpy()) <= TOL
    assert rel_err(ops.norm(x, 1e-5, w=w, b=b), F.layer_norm(t64(x), (n,), t64(w), t64(b), eps=1e-5).numpy()) <= TOL
    assert rel_err(ops.norm(x, 1e-24, rms=True, w=w), F.rms_norm(t64(x), (n,), t64(w), eps=1e-24).numpy()) <= TOL


def test_rms_norm_zero_row_and_scale_invariance(ops):
    x = synth.normal(2, (3, 64), 1.0)
    x[1] = 0.0
    y = ops.norm(x, 1e-24, rms=True)
    assert np.all(y[1] == 0.0)                        # the eps keeps an all-zero row at zero
    y2 = ops.norm(x * 8.0, 1e-24, rms=True)           # exact power-of-two scaling
    assert np.array_equal(y, y2)
    assert np.allclose(np.mean(y[0].astype(np.float64) ** 2), 1.0, atol=1e-6)


# ------------------------------------------------------------------------ SOFT_MAX
@pytest.mark.parametrize("n,scale", [(801, 0.125), (60, 0.125), (7, 1.0), (2048, -0.5), (1, 3.0)])
def test_soft_max_vs_torch(ops, n, scale):
    import torch
    x = synth.normal(n, (5, n), 4.0)
    got = ops.soft_max(x, scale)
    want = torch.softmax(t64(x) * scale, dim=-1).numpy()
    assert rel_err(got, want) <= TOL
    assert np.allclose(got.astype(np.float64).sum(-1), 1.0, atol=1e-6)


def test_soft_max_shift_invariance(ops):
    x = synth.normal(4, (3, 100), 2.0)
    assert rel_err(ops.soft_max(x + 64.0, 0.125), ops.soft_max(x, 0.125)) <= 1e-5


# ---------------------------------------------------------------------------- GELU
def test_gelu_vs_torch_and_identity(ops):
    import torch.nn.functional as F
    x = np.concatenate([synth.normal(11, (100000,), 3.0), np.linspace(-12, 12, 4801, dtype=np.float32)])
    got = ops.gelu(x)
    want = F.gelu(t64(x), approximate="none").numpy()
    assert rel_err(got, want) <= TOL
    # gelu(x) - gelu(-x) = x exactly in real arithmetic.
    d = ops.gelu(x).astype(np.float64) - ops.gelu(-x).astype(np.float64)
    assert np.max(np.abs(d - x) / np.maximum(np.abs(x), 1e-3)) < 1e-6


# ----------------------------------------------------------------------------- GLU
@pytest.mark.parametrize("shape,dim", [((96, 1, 50), 2), ((3, 8, 5, 6), 0), ((4, 10, 3), 1), ((6, 2, 3, 5), 3)])
def test_glu_vs_torch(ops, shape, dim):
    import torch.nn.functional as F
    x = synth.normal(len(shape) + dim, shape, 2.0)
    got = ops.glu(x, dim)
    want = F.glu(t64(x), dim=x.ndim - 1 - dim).numpy()
    assert rel_err(got, want) <= TOL


# ------------------------------------------------------------------ ADD / MUL (exact)
@pytest.mark.parametrize("shape,bshape", [((48, 1, 999), (48, 1, 1)), ((60, 801, 64), (64,)), ((5, 6, 7), (5, 1, 7)),
                                          ((2, 3, 4, 5), (1, 3, 1, 5))])
def test_binary_bit_exact_vs_numpy(ops, shape, bshape):
    a = synth.normal(1, shape, 1.0)
    b = synth.normal(2, bshape, 1.0)
    c = synth.normal(3, bshape, 1e-2)
    bt = np.broadcast_to(b.reshape((1,) * (len(shape) - len(bshape)) + bshape), shape)
    ct = np.broadcast_to(c.reshape((1,) * (len(shape) - len(bshape)) + bshape), shape)
    assert np.array_equal(ops.binary("add", a, b), a + bt)
    assert np.array_equal(ops.binary("mul", a, b), a * bt)
    assert np.array_equal(ops.binary("mul_add", a, b, c), a + (bt * ct))
    assert np.array_equal(ops.binary("add_gelu", a, b), ops.gelu(a + bt))


# ---------------------------------------------------------------------------- ROPE
def rope_complex(x, pos, n_dims, theta=10000.0):
    """Mode 0 as complex multiplication: (x[2k] + i x[2k+1]) * exp(i pos theta^(-2k/d))."""
    x = x.astype(np.float64)
    z = x[..., :n_dims:2] + 1j * x[..., 1:n_dims:2]
    k = np.arange(n_dims // 2)
    ang = pos.astype(np.float64)[:, None] * theta ** (-2.0 * k / n_dims)      # [ne2, k]
    z = z * np.exp(1j * ang)[None, :, None, :] if x.ndim == 4 else z * np.exp(1j * ang)[:, None, :]
    y = x.copy()
    y[..., :n_dims:2] = z.real
    y[..., 1:n_dims:2] = z.imag
    return y


@pytest.mark.parametrize("shape,n_dims", [((3, 37, 8, 64), 64), ((2, 5, 4, 48), 32), ((11, 3, 16), 16)])
def test_rope_vs_complex(ops, shape, n_dims):
    x = synth.normal(7, shape, 1.0)
    ne2 = shape[-3]
    pos = np.arange(ne2, dtype=np.int32) * 3 + 1
    got = ops.rope(x, pos, n_dims)
    want = rope_complex(x, pos, n_dims)
    assert rel_err(got, want) <= TOL


def test_rope_neox_and_invariants(ops):
    x = synth.normal(8, (2, 20, 4, 64), 1.0)
    pos = np.arange(20, dtype=np.int32)
    y = ops.rope(x, pos, 64).astype(np.float64)
    # Pair norms are preserved.
    n_in = x[..., 0::2].astype(np.float64) ** 2 + x[..., 1::2].astype(np.float64) ** 2
    assert np.allclose(y[..., 0::2] ** 2 + y[..., 1::2] ** 2, n_in, rtol=1e-6, atol=1e-12)
    # q.k after RoPE depends only on the position difference: same vectors at (p, p + 3).
    q = np.repeat(x[:1, :1], 20, axis=1)
    yq = ops.rope(q, pos, 64).astype(np.float64)
    dots = [np.sum(yq[0, p] * yq[0, p + 3]) for p in range(17)]
    assert np.ptp(dots) < 1e-4 * np.max(np.abs(dots))
    # NEOX (mode 2) is mode 0 on the de-interleaved layout.
    perm = np.concatenate([np.arange(0, 64, 2), np.arange(1, 64, 2)])
    yn = ops.rope(x[..., perm], pos, 64, mode=2)
    assert rel_err(yn, y[..., perm]) <= TOL
    # Position 0 is the identity; attn_factor scales.
    y0 = ops.rope(x, np.zeros(20, np.int32), 64, attn_factor=2.0)
    assert np.array_equal(y0, 2.0 * x)
