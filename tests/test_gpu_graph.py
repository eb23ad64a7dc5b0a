"""The kernels under HIP graph capture: every entry point launches on the
caller's stream and allocates nothing, so a captured sequence of calls
replays to the same results as eager calls.  Each graph is replayed several
times with eager work and synchronisation in between, and every replay is
compared with the eager output."""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def test_capture_and_replay_matches_eager(gpu):
    import torch

    import kernel_library as kl

    torch.manual_seed(0)
    M, N, K = 512, 768, 1024
    a = torch.empty((K, M), dtype=torch.bfloat16, device=gpu).uniform_(-1, 1)
    lhs = torch.empty((M, K), dtype=torch.bfloat16, device=gpu).uniform_(-1, 1)
    b = torch.empty((K, N), dtype=torch.bfloat16, device=gpu).uniform_(-1, 1)
    x = torch.randn(M, K, device=gpu).bfloat16()
    g = (1 + 0.1 * torch.randn(K, device=gpu)).bfloat16()
    w = (torch.randn(K, N, device=gpu) / 32).bfloat16()
    outs = [torch.empty((M, N), dtype=torch.bfloat16, device=gpu) for _ in range(4)]
    zero_in = torch.empty((0, M), dtype=torch.bfloat16, device=gpu)
    zero_rhs = torch.empty((0, N), dtype=torch.bfloat16, device=gpu)

    def calls():
        kl.matmul_lhsT_rhs(a, b, out=outs[0])
        kl.matmul_lhs_rhs(lhs, b, out=outs[1])
        kl.rmsnorm_matmul(x, w, g, out=outs[2])
        kl.matmul_lhsT_rhs(zero_in, zero_rhs, out=outs[3])   # K = 0: the zero-fill kernel

    calls()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    assert torch.count_nonzero(eager[3]).item() == 0

    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):    # warm-up on the capture stream, as torch requires
        calls()
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        # unrelated eager work between replays
        (b.float() * 2).sum()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), (rep, i)
