"""HIP graph capture of a whole training step (loss + backward): the path launches kernels only
(no memset, no host synchronization, no allocation outside torch's graph pool), so it captures, and
every replay, with new inputs copied into the static tensors and eager work in between, gives the
eager result. Capture removes the host cost of a step (autograd and the launches), which bounds
small volumes."""
import pytest
import torch

import workloads as wl
from fused_lncc import fused_lncc_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream")  # from the side-stream warmup
@pytest.mark.parametrize("target_grad", [False, True])
def test_graph_replays_match_eager(target_grad):
    k = 5
    shape = (1, 2, 24, 30, 36)
    p = torch.zeros(shape, device=DEV, requires_grad=True)
    t = torch.zeros(shape, device=DEV, requires_grad=target_grad)

    def step():
        loss = fused_lncc_loss(p, t, k, target_grad=target_grad)
        loss.backward()
        return loss

    def load(i):
        a, b = wl.randn_pair(shape, 200 + i)
        with torch.no_grad():
            p.copy_(0.6 * b + 0.4 * a)
            t.copy_(b)

    # warm up on a side stream, then capture with the gradients unset (they are created inside
    # the graph, in its memory pool, and rewritten by every replay)
    load(0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            p.grad = None
            t.grad = None
            step()
    torch.cuda.current_stream().wait_stream(s)
    p.grad = None
    t.grad = None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_loss = step()
    gp_static = p.grad
    gt_static = t.grad

    for i in range(1, 5):
        load(i)
        g.replay()
        torch.cuda.synchronize()
        got = (static_loss.item(), gp_static.clone(), gt_static.clone() if target_grad else None)
        # the same step eagerly, on fresh gradients
        saved = (p.grad, t.grad)
        p.grad = None
        t.grad = None
        want_loss = step()
        torch.cuda.synchronize()
        assert got[0] == want_loss.item()
        assert torch.equal(got[1], p.grad)
        if target_grad:
            assert torch.equal(got[2], t.grad)
        p.grad, t.grad = saved
