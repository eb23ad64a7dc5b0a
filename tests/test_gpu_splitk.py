"""GPU parity of split-K (tile config ``split_k`` > 1) for the pipelined lhsT
matmul, against the CPU oracle.

With split_k = P each output tile is computed by P workgroups over disjoint
K ranges; they write fp32 partial products to a workspace that the call
takes from the library's stream-ordered pool (one buffer per call), and a
second kernel sums them in part order into the bf16 output.  The tests
cover ragged M, N and K, part counts up to 8, both pipelined variants,
repeated and interleaved launches of different shapes, a second stream,
run to run determinism, HIP-graph replay, and the pool's cap on the memory
it keeps after large calls.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import mm_check, mm_inputs
from oracle import matmul as omm

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(device)


def _host(t) -> np.ndarray:
    import torch

    return t.to(torch.float32).cpu().numpy()


def _nan_out(M, N, device):
    import torch

    return torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=device)


CONFIGS = [
    # (block_m, block_n, block_k, waves, stages, variant)
    (64, 128, 64, 4, 4, 1),
    (128, 128, 64, 4, 3, 1),
    (256, 256, 32, 4, 3, 1),
    (32, 128, 128, 4, 3, 3),
    (128, 128, 64, 4, 3, 3),
    (128, 128, 64, 4, 4, 4),   # K sub-steps split over the waves
    (128, 128, 32, 2, 4, 4),
]


@pytest.mark.parametrize("parts", [2, 3, 4, 8])
@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: "bm{}_bn{}_bk{}_w{}_s{}_v{}".format(*c))
def test_ragged_shapes_match_oracle(gpu, cfg, parts):
    """M, N not multiples of the block, K not a multiple of block_k (the last part is short)."""
    import kernel_library as kl

    bm, bn, bk, w, s, v = cfg
    M, N, K = 200, 264, 1000
    tc = kl.TileConfig(bm, bn, bk, w, s, split_k=parts, variant=v)
    assert kl.check("matmul_lhsT_rhs", tc, M, N, K)[0] == 0, kl.check("matmul_lhsT_rhs", tc, M, N, K)
    print("split-K", tc.name, M, N, K, flush=True)
    d = mm_inputs(K, M, N, seed=parts)
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    out = _nan_out(M, N, gpu)
    kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    rep = mm_check(_host(out), omm.closed_form(d["lhs_T"], d["rhs"]))
    assert rep["ok"], (tc.name, rep)


def test_interleaved_launches_and_streams(gpu):
    """Interleaved launches with different part counts and shapes on one
    stream, then on a second stream: every output is whole and correct (the
    output starts as NaN, so a part that is not summed shows)."""
    import torch

    import kernel_library as kl

    shapes = [(256, 512, 2048, 4), (136, 128, 512, 2), (256, 512, 2048, 2), (256, 512, 2048, 4),
              (64, 1024, 4096, 8)]
    data = {}
    for M, N, K, _ in shapes:
        if (M, N, K) not in data:
            d = mm_inputs(K, M, N, seed=M + N + K)
            data[(M, N, K)] = (d, _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu))
    side = torch.cuda.Stream(device=gpu)
    for stream in (torch.cuda.current_stream(gpu), side):
        with torch.cuda.stream(stream):
            for rep_i in range(2):
                for M, N, K, parts in shapes:
                    d, a, b = data[(M, N, K)]
                    tc = kl.TileConfig(64, 128, 64, 4, 4, split_k=parts, variant=1)
                    out = _nan_out(M, N, gpu)
                    kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
                    stream.synchronize()
                    rep = mm_check(_host(out), omm.closed_form(d["lhs_T"], d["rhs"]))
                    assert rep["ok"], (M, N, K, parts, rep_i, rep)
    torch.cuda.synchronize()


def test_deterministic_and_close_to_unsplit(gpu):
    """The same split call twice gives the same bits (parts are summed in a
    fixed order); against the unsplit kernel the difference is fp32
    summation order only."""
    import torch

    import kernel_library as kl

    M, N, K = 512, 512, 8192
    d = mm_inputs(K, M, N, seed=11)
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    split = kl.TileConfig(128, 128, 64, 4, 3, split_k=4, variant=1)
    whole = kl.TileConfig(128, 128, 64, 4, 3, variant=1)
    outs = [kl.matmul_lhsT_rhs(a, b, cfg=split) for _ in range(3)]
    ref = kl.matmul_lhsT_rhs(a, b, cfg=whole)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    diff = (outs[0].float() - ref.float()).abs().max().item()
    scale = ref.float().abs().max().item()
    assert diff <= 2 ** -7 * scale, (diff, scale)
    rep = mm_check(_host(outs[0]), omm.closed_form(d["lhs_T"], d["rhs"]))
    assert rep["ok"], rep


@pytest.mark.parametrize("M,N,K,cfg", [
    (2048, 1024, 8192, (128, 128, 64, 4, 3, 1, 2)),   # benchmark config C4a, 128 tiles x 2 parts
    (128, 28672, 8192, (128, 128, 64, 4, 2, 3, 2)),   # C5 at M = 128, 224 tiles x 2 parts
    (256, 512, 32768, (128, 128, 64, 4, 3, 1, 16)),   # 8 output tiles, long K: 16 parts
])
def test_benchmark_shapes(gpu, M, N, K, cfg):
    """Split-K configs at shapes with few output tiles, whole output vs the oracle."""
    import kernel_library as kl

    bm, bn, bk, w, s, v, p = cfg
    tc = kl.TileConfig(bm, bn, bk, w, s, split_k=p, variant=v)
    print("split-K", tc.name, M, N, K, flush=True)
    d = mm_inputs(K, M, N, seed=0)
    out = _nan_out(M, N, gpu)
    kl.matmul_lhsT_rhs(_dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu), cfg=tc, out=out)
    rep = mm_check(_host(out), omm.closed_form(d["lhs_T"], d["rhs"]))
    assert rep["ok"], (tc.name, rep)


def test_concurrent_streams(gpu):
    """Split-K calls on two streams with no synchronisation between them: each call has its own workspace."""
    import torch

    import kernel_library as kl

    M, N, K = 256, 512, 8192
    tc = kl.TileConfig(64, 128, 64, 4, 4, split_k=8, variant=1)
    ds = [mm_inputs(K, M, N, seed=30 + i) for i in range(2)]
    ins = [(_dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)) for d in ds]
    streams = [torch.cuda.Stream(device=gpu) for _ in range(2)]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream(gpu))
    outs = [[None] * 4 for _ in range(2)]
    for rep_i in range(4):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                outs[i][rep_i] = kl.matmul_lhsT_rhs(*ins[i], cfg=tc)
    torch.cuda.synchronize()
    for i, d in enumerate(ds):
        expected = omm.closed_form(d["lhs_T"], d["rhs"])
        for rep_i in range(4):
            rep = mm_check(_host(outs[i][rep_i]), expected)
            assert rep["ok"], (i, rep_i, rep)


def test_graph_replay_matches_eager(gpu):
    """A split-K call captured in a HIP graph (its workspace becomes allocation
    and free nodes of the graph) replays to the eager result, with eager
    split-K work between replays."""
    import torch

    import kernel_library as kl

    M, N, K = 256, 384, 4096
    d = mm_inputs(K, M, N, seed=5)
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    tc = kl.TileConfig(64, 128, 64, 4, 4, split_k=4, variant=1)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    for rep_i in range(4):
        out.fill_(float("nan"))
        kl.matmul_lhsT_rhs(a, b, cfg=tc)          # eager split-K work on the current stream between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), rep_i


def test_library_default_splits_few_tile_long_k(gpu):
    """With no config and no tuned entry, a few-tile long-K shape takes a split-K default; output vs the oracle."""
    import kernel_library as kl

    M, N, K = 512, 256, 16384
    cfg = kl.default_config("matmul_lhsT_rhs", M, N, K)
    assert cfg.split_k > 1, cfg
    d = mm_inputs(K, M, N, seed=9)
    out = kl.matmul_lhsT_rhs(_dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu))
    rep = mm_check(_host(out), omm.closed_form(d["lhs_T"], d["rhs"]))
    assert rep["ok"], (cfg.name, rep)


@pytest.mark.parametrize("parts", [2, 4])
@pytest.mark.parametrize("cfg", [(128, 128, 64, 4, 3, 0), (256, 256, 32, 4, 3, 0), (64, 128, 64, 4, 4, 2)],
                         ids=lambda c: "bm{}_bn{}_bk{}_w{}_s{}_v{}".format(*c))
def test_lhs_rhs_split_matches_oracle_and_lhsT(gpu, cfg, parts):
    """matmul_lhs_rhs (K-contiguous lhs) with split-K: ragged M, N and K vs the oracle, and bitwise equal to
    the lhsT kernel's split-K on the transposed operand (same K parts, same MFMA order)."""
    import torch

    import kernel_library as kl

    bm, bn, bk, w, s, v = cfg
    M, N, K = 200, 264, 1000
    tc = kl.TileConfig(bm, bn, bk, w, s, split_k=parts, variant=v)
    print("split-K lhs", tc.name, M, N, K, flush=True)
    d = mm_inputs(K, M, N, seed=20 + parts)
    lhs = _dev(np.ascontiguousarray(d["lhs_T"].T), gpu)
    rhs = _dev(d["rhs"], gpu)
    out = _nan_out(M, N, gpu)
    kl.matmul_lhs_rhs(lhs, rhs, cfg=tc, out=out)
    rep = mm_check(_host(out), omm.closed_form_lhs(np.ascontiguousarray(d["lhs_T"].T), d["rhs"]))
    assert rep["ok"], (tc.name, rep)
    twin = kl.TileConfig(bm, bn, bk, w, s, split_k=parts, variant=1 if v == 0 else 3)
    ref = kl.matmul_lhsT_rhs(_dev(d["lhs_T"], gpu), rhs, cfg=twin)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (tc.name, twin.name)


@pytest.mark.parametrize("with_gamma", [True, False])
@pytest.mark.parametrize("parts", [2, 4])
@pytest.mark.parametrize("cfg,K", [((128, 128, 64, 4, 2, 4), 1000), ((128, 512, 32, 8, 3, 4), 1000),
                                   ((256, 256, 32, 8, 3, 5), 1000), ((128, 128, 32, 4, 3, 12), 1000),
                                   ((64, 128, 64, 4, 2, 11), 1000), ((128, 128, 64, 4, 3, 13), 1000),
                                   ((256, 256, 32, 4, 3, 13), 1000), ((128, 128, 64, 4, 3, 13), 5000),
                                   ((64, 128, 64, 4, 4, 13), 5000)],
                         ids=lambda c: "bm{}_bn{}_bk{}_w{}_s{}_v{}".format(*c) if isinstance(c, tuple) else f"K{c}")
def test_rmsnorm_split_matches_oracle(gpu, cfg, K, parts, with_gamma):
    """Fused rmsnorm_matmul with split-K: each part's products and row sums of
    squares are summed by the second pass, which applies 1/rms.  Ragged M, N,
    K (a multiple of 8, not of block_k); a zero row stays exactly zero.  The
    two-pass kernel (variant 13) splits its core and hands the second pass
    the pack's row sums of squares, one per 512 columns of K: 2 at K = 1000,
    10 at K = 5000 (more than the 8 the unsplit core sums per load)."""
    import kernel_library as kl
    from helpers import rms_check, rms_inputs
    from oracle import rmsnorm as orms

    bm, bn, bk, w, s, v = cfg
    M, N = 200, 264
    tc = kl.TileConfig(bm, bn, bk, w, s, split_k=parts, variant=v)
    print("split-K rms", tc.name, M, N, K, with_gamma, flush=True)
    d = rms_inputs(M, K, N, seed=40 + parts, with_gamma=with_gamma)
    x = d["lhs"].copy()
    x[5] = 0.0
    g = _dev(d["gamma"], gpu) if with_gamma else None
    out = _nan_out(M, N, gpu)
    kl.rmsnorm_matmul(_dev(x, gpu), _dev(d["rhs"], gpu), g, cfg=tc, out=out)
    host = _host(out)
    rep = rms_check(host, orms.closed_form(x, d["rhs"], d["gamma"] if with_gamma else None))
    assert rep["ok"], (tc.name, rep)
    assert np.all(host[5] == 0.0)


def test_rmsnorm_split_lifts_the_gamma_limit(gpu):
    """K = 16384 is past the 8192 fp32 gamma entries a register-staged kernel
    holds in LDS; split in two, each part stages 8192."""
    import kernel_library as kl
    from helpers import rms_check, rms_inputs
    from oracle import rmsnorm as orms

    M, K, N = 256, 16384, 1024
    whole = kl.TileConfig(128, 128, 64, 4, 2, variant=4)
    split = kl.TileConfig(128, 128, 64, 4, 2, split_k=2, variant=4)
    assert kl.check("rmsnorm_matmul", whole, M, N, K)[0] != 0
    assert kl.check("rmsnorm_matmul", split, M, N, K)[0] == 0
    d = rms_inputs(M, K, N, seed=44)
    out = kl.rmsnorm_matmul(_dev(d["lhs"], gpu), _dev(d["rhs"], gpu), _dev(d["gamma"], gpu), cfg=split)
    rep = rms_check(_host(out), orms.closed_form(d["lhs"], d["rhs"], d["gamma"]))
    assert rep["ok"], rep


@pytest.mark.parametrize("M,K,N", [(256, 16384, 1024), (16, 16384, 4096), (4096, 16384, 7168)])
def test_rmsnorm_default_past_the_gamma_limit(gpu, M, K, N):
    """With no config and K > 8192: few output tiles or skinny M take a split
    register-staged fused config (each part's gamma in LDS); many output tiles
    take the two-pass kernel (no gamma limit, no split).  Output vs the oracle (sampled rows at the
    large shape), and at the large shape the default against variant 0 (the
    other config without a gamma limit), timed."""
    import torch

    import kernel_library as kl
    from autotune.runner.benchmark import time_launches
    from helpers import rms_check, rms_inputs
    from oracle import rmsnorm as orms

    print(f"fused default M={M} K={K} N={N}", flush=True)
    cfg = kl.default_config("rmsnorm_matmul", M, N, K)
    big = M * N >= 2048 * 2048
    if big:
        assert cfg.variant == 13 and cfg.split_k == 1, cfg
    else:
        assert cfg.split_k > 1 and cfg.variant in (4, 5, 11), cfg
    d = rms_inputs(M, K, N, seed=45)
    x, w, g = _dev(d["lhs"], gpu), _dev(d["rhs"], gpu), _dev(d["gamma"], gpu)
    out = kl.rmsnorm_matmul(x, w, g)
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(2).integers(0, M, size=min(M, 20))]))
    rep = rms_check(_host(out)[rows], orms.closed_form(d["lhs"][rows], d["rhs"], d["gamma"]))
    assert rep["ok"], (cfg.name, rep)
    if big:
        v0 = kl.TileConfig(128, 256, 64, 8, 2, variant=0)
        o0 = torch.empty_like(out)
        t13 = sorted(time_launches(lambda: kl.rmsnorm_matmul(x, w, g, cfg=cfg, out=out), 2, 10))[5]
        t0 = sorted(time_launches(lambda: kl.rmsnorm_matmul(x, w, g, cfg=v0, out=o0), 2, 10))[5]
        print(f"default {cfg.name} {t13 * 1e6:.0f} us, variant 0 {v0.name} {t0 * 1e6:.0f} us", flush=True)
        rep0 = rms_check(_host(o0)[rows], orms.closed_form(d["lhs"][rows], d["rhs"], d["gamma"]))
        assert rep0["ok"], rep0
        # The timing is reported, not gated, beyond a margin that only a
        # broken default would exceed (clocks vary between runs and boxes).
        assert t13 < 1.5 * t0


def test_pool_returns_memory_after_a_large_call(gpu):
    """A split-K call whose workspace is 1 GiB, then a synchronisation: the
    runtime hands the freed buffer back to the library's pool only at the
    pool's next allocation (the figure is printed), and
    ``release_workspace`` returns it, so the device's free memory is back to
    its level before the call."""
    import torch

    import kernel_library as kl

    M = N = 8192
    K = 16384
    tc = kl.TileConfig(256, 256, 32, 4, 3, split_k=4, variant=1)      # 4 x 8192 x 8192 x 4 B = 1 GiB
    a = torch.zeros((K, M), dtype=torch.bfloat16, device=gpu)
    b = torch.zeros((K, N), dtype=torch.bfloat16, device=gpu)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    torch.cuda.synchronize()
    kl.release_workspace()
    free_before = torch.cuda.mem_get_info(gpu)[0]
    kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    torch.cuda.synchronize()
    torch.cuda.synchronize()
    held = free_before - torch.cuda.mem_get_info(gpu)[0]
    print(f"pool holds {held / 2**20:.0f} MiB after a 1 GiB workspace call and two synchronisations", flush=True)
    kl.release_workspace()
    held = free_before - torch.cuda.mem_get_info(gpu)[0]
    print(f"pool holds {held / 2**20:.0f} MiB after release_workspace", flush=True)
    assert held <= 32 << 20, held
    assert torch.count_nonzero(out).item() == 0
