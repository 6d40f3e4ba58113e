"""ovg_op_linear_noalloc (the no-allocation variant of ovg_op_linear, with
its split-K partials in a static device array) gives ovg_op_linear's result
bit for bit: two calls in a row, the second on a smaller input, both at
shapes whose plan splits K (so the static array is used and reused)."""
import numpy as np
import pytest

import omnivoice_amd as ov

pytestmark = pytest.mark.gpu


def _torch_gpu():
    try:
        import torch
        return torch if torch.cuda.is_available() else None
    except Exception:
        return None


@pytest.fixture(scope="module")
def torch():
    t = _torch_gpu()
    if t is None:
        pytest.skip("no GPU")
    return t


def test_linear_noalloc_matches_linear(torch):
    gen = torch.Generator().manual_seed(11)
    # (rows, in, out, accumulate): 8 and 4 K-splits of 32-row tiles.
    for rows, k, n, acc in [(40, 2048, 512, False), (17, 1024, 256, True)]:
        x = (torch.randn(rows, k, generator=gen) * 0.5).half().cuda()
        w = (torch.randn(n, k, generator=gen) * 0.05).half().cuda()
        y0 = torch.randn(rows, n, generator=gen).cuda()
        want = y0.clone()
        ov.op_linear(x, w, want, accumulate=acc)
        got = y0.clone()
        ov.op_linear_noalloc(x, w, got, accumulate=acc)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (rows, k, n)
        ref = x.float() @ w.float().t() + (y0 if acc else 0)
        assert torch.allclose(got, ref, rtol=1e-3, atol=1e-3)


def test_linear_noalloc_captured_in_a_graph(torch):
    """After a first eager call on the device (which looks up the array's
    address), the entry point captured in a graph on a side stream replays
    to ovg_op_linear's result bit for bit, replay after replay, with other
    eager work between the replays."""
    gen = torch.Generator().manual_seed(12)
    rows, k, n = 40, 2048, 512  # 32-row tiles in 8 K-splits: the array is used
    x = (torch.randn(rows, k, generator=gen) * 0.5).half().cuda()
    w = (torch.randn(n, k, generator=gen) * 0.05).half().cuda()
    want = torch.empty(rows, n, device="cuda")
    ov.op_linear(x, w, want)
    warm = torch.empty(rows, n, device="cuda")
    ov.op_linear_noalloc(x, w, warm)
    torch.cuda.synchronize()
    assert torch.equal(warm, want)
    got = torch.empty(rows, n, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            ov.op_linear_noalloc(x, w, got, stream=side)
    torch.cuda.current_stream().wait_stream(side)
    other = (torch.randn(rows, k, generator=gen) * 0.5).half().cuda()
    for replay in range(3):
        got.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), replay
        # Eager work on the same array between replays.
        scratch_user = torch.empty(rows, n, device="cuda")
        ov.op_linear_noalloc(other, w, scratch_user)
        torch.cuda.synchronize()
