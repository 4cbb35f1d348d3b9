"""CPU checks that pin the layout oracle (oracle/layout_oracle.c).

ggml_permute's axis meaning is fixed by the reference's own comments on its permutes
(src/roformer.cpp:112-114, :133, :182, :184): those shapes are asserted here. Element placement
is checked bit for bit against numpy's transpose and concatenate (an independent statement of
the same data movement), and the q/k/v split against the complex-multiplication RoPE on numpy's
slices of qkv, so a wrong head offset, a swapped permute or a dropped rotation fails.
"""
import itertools

import numpy as np
import pytest

import oracle_lib
import synth
from metrics import rel_err
from test_oracle_ops import rope_complex

TOL = 1e-6


@pytest.fixture(scope="module")
def ops():
    return oracle_lib.ops()


def np_permute(x, axes):
    """ggml_cont(ggml_permute(x, axes)) in numpy: ggml dim i of x -> ggml dim axes[i] of y; numpy
    axis of ggml dim g is (3 - g) for a 4-d array."""
    x4 = x.reshape((1,) * (4 - x.ndim) + x.shape)
    perm = [0] * 4
    for i, a in enumerate(axes):
        perm[3 - a] = 3 - i
    return np.ascontiguousarray(np.transpose(x4, perm))


def test_reference_permute_shapes(ops):
    dh, H, N, B = 5, 3, 7, 2
    part = np.zeros((B, N, H, dh), np.float32)                    # ggml [dh, H, N, batch]
    assert ops.cont_permute(part, (0, 2, 1, 3)).shape == (B, H, N, dh)    # [dh, N, H, batch] :112
    assert ops.cont_permute(part, (1, 2, 0, 3)).shape == (B, H, dh, N)    # [N, dh, H, batch] :114
    x = np.zeros((1, 11, 4, 6), np.float32)                      # ggml [D, B, T]
    assert ops.cont_permute(x, (0, 2, 1, 3)).shape == (1, 4, 11, 6)       # [D, T, B] :182


@pytest.mark.parametrize("axes", list(itertools.permutations(range(4))))
def test_cont_permute_vs_numpy(ops, axes):
    x = synth.normal(3, (2, 3, 5, 7), 1.0)
    got = ops.cont_permute(x, axes)
    assert np.array_equal(got, np_permute(x, axes))


def test_cont_permute_element_placement(ops):
    # x[i3, i2, i1, i0] = a distinct code; (1,2,0,3) sends (i0, i1, i2) to (i1, i2, i0).
    x = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    y = ops.cont_permute(x, (1, 2, 0, 3))
    assert y.shape == (2, 4, 5, 3)
    for i3, i2, i1, i0 in itertools.product(range(2), range(3), range(4), range(5)):
        assert y[i3, i1, i0, i2] == x[i3, i2, i1, i0]


@pytest.mark.parametrize("dim", [0, 1, 2, 3])
def test_concat_vs_numpy(ops, dim):
    base = [3, 4, 5, 6]
    xs = []
    for s, extent in enumerate([1, 4, 2]):
        shape = list(base)
        shape[3 - dim] = extent
        xs.append(synth.normal(10 + s, tuple(shape), 1.0))
    got = ops.concat(xs, dim)
    assert np.array_equal(got, np.concatenate(xs, axis=3 - dim))


def test_concat_tree_equals_flat(ops):
    """concat_all's balanced tree of pairwise concats (src/roformer.cpp:52-60) places every
    source where one flat concat does."""
    xs = [synth.normal(20 + i, (7, 1, 6), 1.0) for i in range(7)]
    v = list(xs)
    while len(v) > 1:
        nxt = [ops.concat([v[i], v[i + 1]], 1) for i in range(0, len(v) - 1, 2)]
        if len(v) % 2:
            nxt.append(v[-1])
        v = nxt
    assert np.array_equal(v[0], ops.concat(xs, 1))


@pytest.mark.parametrize("B,N,H,dh", [(2, 9, 3, 8), (3, 5, 2, 64), (1, 70, 1, 32)])
def test_qkv_rope_split_vs_numpy(ops, B, N, H, dh):
    qkv = synth.normal(5, (B, N, 3 * H * dh), 1.0)
    pos = (np.arange(N, dtype=np.int32) * 7 + 3) % 101
    q, k, vt = ops.qkv_rope_split(qkv, pos, H, freq_base=10000.0)
    for i, got in enumerate((q, k)):
        part = qkv[:, :, i * H * dh:(i + 1) * H * dh].reshape(B, N, H, dh)      # ggml [dh, H, N, B]
        want = rope_complex(part, pos, dh)                                       # rotates by N (ggml ne2)
        assert rel_err(got, np.transpose(want, (0, 2, 1, 3))) <= TOL
    v = qkv[:, :, 2 * H * dh:].reshape(B, N, H, dh)
    assert np.array_equal(vt, np.ascontiguousarray(np.transpose(v, (0, 2, 3, 1))))


def test_qkv_rope_split_scales(ops):
    qkv = synth.normal(6, (2, 4, 3 * 2 * 16), 1.0)
    pos = np.zeros(4, np.int32)
    q, k, _ = ops.qkv_rope_split(qkv, pos, 2, attn_factor=2.0)
    part = qkv[:, :, :32].reshape(2, 4, 2, 16)
    assert np.array_equal(q, 2.0 * np.transpose(part, (0, 2, 1, 3)))


def test_merge_heads_vs_numpy(ops):
    o = synth.normal(7, (3, 4, 9, 8), 1.0)                     # (batch, H, N, dh)
    g = synth.normal(8, (3, 9, 4), 1.0)                        # (batch, N, H)
    y = ops.merge_heads(o)
    assert np.array_equal(y, np.ascontiguousarray(np.transpose(o, (0, 2, 1, 3))))
    yg = ops.merge_heads(o, g)
    assert np.array_equal(yg, np.transpose(o, (0, 2, 1, 3)) * g[..., None])
