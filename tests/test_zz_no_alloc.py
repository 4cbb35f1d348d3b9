"""stx_group_norm_noalloc, the group norm that takes its scratch from the library's static
per-GPU array instead of a workspace, against stx_group_norm with a workspace (the same kernels
and the same statistics order: the outputs must be the same bits), through the C ABI.

Two calls in a row on the shared scratch, the second on a smaller input, for the single-pass
shapes (C = 48 then C = 384 of the HTDemucs op set) and for the two-pass path (in place, and
many groups); a shape whose scratch would exceed STX_GROUP_NORM_SCRATCH_BYTES is refused.
"""
import numpy as np
import pytest

import oracle_lib
import stx
from metrics import rel_err

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 1 << 20              # STX_GROUP_NORM_SCRATCH_BYTES


def randn(device, shape, seed, sigma=1.0, mean=0.0):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32) * sigma + mean


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("calls", [
    [((48, 1, 85995), 1, True), ((384, 1, 1344), 1, True)],            # single pass, larger then smaller
    [((96, 1, 21499), 1, False), ((8, 1, 3000), 4, False)],
    [((1000, 1, 8192), 1000, True), ((200, 1, 4000), 50, True)],        # two passes (many groups)
])
def test_noalloc_matches_workspace_entry_point(device, calls):
    ops = oracle_lib.ops()
    for shape, G, gelu in calls:
        x = randn(device, shape, sum(shape), 1.2, 0.4)
        C = shape[-3]
        w, b = randn(device, (C, 1, 1), 80), randn(device, (C, 1, 1), 81)
        assert stx.group_norm_workspace_size(x, G) <= SCRATCH_BYTES
        want = host(stx.group_norm(x, G, 1e-5, w, b, gelu=gelu))
        got = host(stx.group_norm_noalloc(x, G, 1e-5, w, b, gelu=gelu))
        assert np.array_equal(got, want)
        assert rel_err(got, ops.group_norm(host(x), G, 1e-5, host(w), host(b), gelu=gelu)) <= 1e-6


def test_noalloc_in_place_and_graph_replays(device):
    """In place (two passes on the scratch), then replays of a captured call on new data."""
    import torch
    C, T = 96, 21499
    x = randn(device, (C, 1, T), 90)
    w, b = randn(device, (C, 1, 1), 91), randn(device, (C, 1, 1), 92)
    want = host(stx.group_norm(x, 1, 1e-5, w, b, gelu=True))
    xc = x.clone()
    stx.group_norm_noalloc(xc, 1, 1e-5, w, b, gelu=True, out=xc)
    assert np.array_equal(host(xc), want)
    y = torch.empty_like(x)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        stx.group_norm_noalloc(x, 1, 1e-5, w, b, gelu=True, out=y, stream=s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            stx.group_norm_noalloc(x, 1, 1e-5, w, b, gelu=True, out=y, stream=s)
    torch.cuda.synchronize()
    for rep in range(3):
        x.copy_(randn(device, (C, 1, T), 93 + rep, 1.0 + rep))
        torch.cuda.synchronize()
        g.replay()
        assert np.array_equal(host(y), host(stx.group_norm(x, 1, 1e-5, w, b, gelu=True)))


def test_noalloc_refuses_shapes_beyond_the_scratch(device):
    x = randn(device, (30000, 1, 64), 95)
    assert stx.group_norm_workspace_size(x, 30000) > SCRATCH_BYTES
    with pytest.raises(stx.StxError) as e:
        stx.group_norm_noalloc(x, 30000)
    assert e.value.status == stx.STATUS_INVALID_ARGUMENT and "static" in str(e.value)
