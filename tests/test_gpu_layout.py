"""GPU parity of the layout glue (layout.hip) against the oracle.

Bar: bit-exact for every pure data movement (vt, the permutes, concat, the head merge and its
gate multiply, which rounds once like ggml_mul); q and k within rel_err <= 1e-6 of the oracle's
RoPE (evaluated in double) and bit-exact against stx_rope_ext on the same view followed by the
permute, which is the node chain the fused kernel replaces.

Shapes: the RoFormer attention of 384 = 8 x 64 over the time axis (qkv [1536, 801, 60]) and the
band axis (qkv [1536, 60, 801]) (ggml order; numpy shapes below are reversed), plus small and
ragged ones (N not a multiple of the 64-position tile, one head, dh 32 and 128, strided qkv).
"""
import itertools

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


def randn(device, shape, seed, sigma=1.0):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32) * sigma


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rope_chain(qkv, pos, H, i, **kw):
    """part(i) = cont(view), rope_ext, cont(permute(0,2,1,3)) through the library's own nodes."""
    B, N, width = qkv.shape
    dh = width // (3 * H)
    part = qkv[:, :, i * H * dh:(i + 1) * H * dh].reshape(B, N, H, dh).contiguous()
    r = stx.rope_ext(part, pos, dh, **kw)
    return stx.cont_permute(r, (0, 2, 1, 3))


QKV_CASES = [
    # batch, N, H, dh
    (60, 801, 8, 64),       # time axis
    (801, 60, 8, 64),       # band axis
    (3, 65, 2, 64),
    (2, 1, 1, 64),
    (5, 63, 3, 32),
    (2, 130, 2, 128),
    (1, 64, 8, 64),
]


@pytest.mark.parametrize("B,N,H,dh", QKV_CASES)
def test_qkv_rope_split(device, ops, B, N, H, dh):
    import torch
    qkv = randn(device, (B, N, 3 * H * dh), B * 1000 + N)
    posh = np.arange(N, dtype=np.int32)
    pos = torch.from_numpy(posh).to(device)
    q, k, vt = stx.qkv_rope_split(qkv, pos, H, freq_base=10000.0)
    print(f"qkv_rope_split B={B} N={N} H={H} dh={dh}", flush=True)
    wq, wk, wvt = ops.qkv_rope_split(host(qkv), posh, H, freq_base=10000.0)
    assert np.array_equal(host(vt), wvt)
    assert rel_err(host(q), wq) <= TOL
    assert rel_err(host(k), wk) <= TOL
    if B * N * H * dh <= 8_000_000:
        assert np.array_equal(host(q), host(rope_chain(qkv, pos, H, 0)))
        assert np.array_equal(host(k), host(rope_chain(qkv, pos, H, 1)))


def test_qkv_rope_split_params_and_strides(device, ops):
    """Arbitrary positions, freq parameters, and a qkv view whose rows are wider than 3*H*dh."""
    import torch
    B, N, H, dh = 4, 77, 3, 64
    big = randn(device, (B, N, 3 * H * dh + 12), 11)
    qkv = big[:, :, 4:4 + 3 * H * dh]                     # 16-byte aligned start, padded rows
    posh = ((np.arange(N, dtype=np.int64) * 7919) % 5000).astype(np.int32)
    pos = torch.from_numpy(posh).to(device)
    kw = dict(freq_base=500.0, freq_scale=0.25, attn_factor=1.5)
    q, k, vt = stx.qkv_rope_split(qkv, pos, H, **kw)
    wq, wk, wvt = ops.qkv_rope_split(host(qkv), posh, H, **kw)
    assert np.array_equal(host(vt), wvt)
    assert rel_err(host(q), wq) <= TOL
    assert rel_err(host(k), wk) <= TOL
    assert np.array_equal(host(q), host(rope_chain(qkv, pos, H, 0, **kw)))


def test_qkv_rope_split_errors(device):
    import torch
    pos = torch.arange(5, dtype=torch.int32, device=device)
    qkv = randn(device, (2, 5, 3 * 2 * 48), 1)
    with pytest.raises(stx.StxError) as e:
        stx.qkv_rope_split(qkv, pos, 2)
    assert e.value.status == stx.STATUS_UNSUPPORTED
    qkv = randn(device, (2, 5, 3 * 2 * 64), 1)
    q = torch.empty((2, 2, 5, 64), device=device)
    with pytest.raises(stx.StxError) as e:                      # wrong vt shape
        stx.qkv_rope_split(qkv, pos, 2, out=(q, torch.empty_like(q), torch.empty_like(q)))
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT
    flat = randn(device, (2 * 5 * 3 * 2 * 64 + 1,), 2)
    with pytest.raises(stx.StxError):                           # rows not 16-byte aligned
        stx.qkv_rope_split(flat[1:].view(2, 5, 3 * 2 * 64), pos, 2)


MERGE_CASES = [(60, 8, 801, 64), (801, 8, 60, 64), (3, 5, 7, 6), (2, 1, 33, 64)]


@pytest.mark.parametrize("B,H,N,dh", MERGE_CASES)
@pytest.mark.parametrize("gated", [False, True])
def test_merge_heads(device, ops, B, H, N, dh, gated):
    o = randn(device, (B, H, N, dh), B + H + N)
    g = None
    if gated:
        import torch
        g = torch.sigmoid(randn(device, (B, N, H, 1), 5))
    y = stx.merge_heads(o, g)
    want = ops.merge_heads(host(o), None if g is None else host(g)[..., 0])
    assert np.array_equal(host(y), want)


@pytest.mark.parametrize("axes", list(itertools.permutations(range(4))))
@pytest.mark.parametrize("shape", [(3, 5, 7, 9), (2, 3, 66, 68)])
def test_cont_permute_all_axes(device, ops, axes, shape):
    x = randn(device, shape, sum(shape))
    y = stx.cont_permute(x, axes)
    assert np.array_equal(host(y), ops.cont_permute(host(x), axes))


@pytest.mark.parametrize("shape,axes", [((801, 60, 384), (0, 2, 1, 3)), ((60, 801, 384), (0, 2, 1, 3)),
                                        ((60, 8, 801, 64), (1, 2, 0, 3)), ((8, 801, 60, 64), (2, 0, 1, 3))])
def test_cont_permute_roformer(device, ops, shape, axes):
    """The transformer's [D, B, T] <-> [D, T, B] transposes (src/roformer.cpp:182,184,190) and the
    v permute (:114) at full size."""
    x = randn(device, shape, 3)
    y = stx.cont_permute(x, axes)
    assert np.array_equal(host(y), ops.cont_permute(host(x), axes))


def test_cont_permute_strided_source(device, ops):
    big = randn(device, (6, 10, 72), 4)
    x = big[1:5, 2:9, 4:68]                                   # strided view, 16-byte aligned rows
    for axes in [(0, 2, 1, 3), (1, 0, 2, 3), (2, 1, 0, 3)]:
        y = stx.cont_permute(x, axes)
        assert np.array_equal(host(y), ops.cont_permute(host(x.contiguous()), axes))


def test_cont_permute_errors(device):
    import torch
    x = randn(device, (3, 4, 5), 1)
    with pytest.raises(stx.StxError):
        stx.cont_permute(x, (0, 0, 1, 2))
    with pytest.raises(stx.StxError):
        stx.cont_permute(x, (0, 2, 1, 3), out=torch.empty((3, 4, 5), device=device))
    with pytest.raises(stx.StxError):                          # dst overlapping src
        stx.cont_permute(x, (0, 1, 2, 3), out=x)


def test_concat_band_split(device, ops):
    """concat_all of the 60 band-split outputs [384, 1, 801] along dim 1 (src/roformer.cpp:178)."""
    xs = [randn(device, (801, 1, 384), 100 + b) for b in range(60)]
    y = stx.concat(xs, 1)
    assert np.array_equal(host(y), ops.concat([host(x) for x in xs], 1))


@pytest.mark.parametrize("dim", [0, 1, 2, 3])
def test_concat_dims(device, ops, dim):
    base = [2, 3, 5, 7]
    xs = []
    for s, extent in enumerate([3, 1, 4, 2, 0, 5]):
        shape = list(base)
        shape[3 - dim] = extent
        xs.append(randn(device, tuple(shape), 10 + s))
    y = stx.concat(xs, dim)
    assert np.array_equal(host(y), ops.concat([host(x) for x in xs], dim))


def test_concat_many_sources_aligned(device, ops):
    """More sources than one launch carries, float4 path, and attention batch groups along dim 3."""
    xs = [randn(device, (1 + (s % 3), 8, 9, 64), 200 + s) for s in range(70)]
    y = stx.concat(xs, 3)
    assert np.array_equal(host(y), ops.concat([host(x) for x in xs], 3))


def test_concat_errors(device):
    a = randn(device, (2, 3), 1)
    b = randn(device, (2, 4), 2)
    with pytest.raises(stx.StxError):
        stx.concat([a, b], 1)
