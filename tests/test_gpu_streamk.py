"""GPU parity of the stream-K lhsT.rhs matmul (variants 5 and 6) against the oracle.

A stream-K launch runs one workgroup per CU; each takes an equal share of
every output tile's K loop, so most tiles are computed in parts by two or
more workgroups, which hand fp32 partial sums to each other through the
workspace and a counter per tile (csrc/mi_streamk.hpp).  The tests cover
ragged shapes, tiles split into many parts (one K tile per workgroup, so
the parts race and every branch of the combine protocol runs), the skinny
benchmark shapes C5 at full size against a float64 product, run-to-run
determinism (the combiner sums in a fixed part order), counters left at
zero for the next call, two streams at once (each with its kept
workspace), HIP-graph replay (a workspace of its own whose counters a
small kernel zeroes) and the no-allocation entry point.  Every output
starts as NaN, so a tile that no part stores shows.
"""

from __future__ import annotations

import ctypes

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


def _f64_check(out, a, b):
    """The whole output against a float64 product of the same bf16 inputs on the GPU."""
    exp = (a.double().t() @ b.double()).cpu().numpy()
    return mm_check(_host(out), exp)


SK_CONFIGS = [
    # (block_m, block_n, block_k, waves, stages, variant)
    (32, 128, 128, 4, 3, 6),
    (64, 128, 64, 4, 4, 6),
    (128, 128, 64, 4, 3, 6),
    (128, 128, 64, 4, 4, 5),
    (32, 256, 64, 4, 4, 5),
    (64, 256, 64, 4, 3, 6),
]


@pytest.mark.parametrize("cfg", SK_CONFIGS, ids=lambda c: "bm{}_bn{}_bk{}_w{}_s{}_v{}".format(*c))
@pytest.mark.parametrize("shape", [(200, 264, 1000), (96, 3000, 2056), (128, 256, 8192)],
                         ids=lambda s: "M{}_N{}_K{}".format(*s))
def test_streamk_matches_oracle(gpu, cfg, shape):
    """Ragged M and N, K not a multiple of block_k; the last shape has one or
    two output tiles over 128 K tiles, so each tile is cut into up to 128
    parts of one K tile each."""
    import kernel_library as kl

    M, N, K = shape
    bm, bn, bk, w, s, v = cfg
    tc = kl.TileConfig(bm, bn, bk, w, s, variant=v)
    assert kl.check("matmul_lhsT_rhs", tc, M, N, K)[0] == 0, kl.check("matmul_lhsT_rhs", tc, M, N, K)
    print("stream-K", tc.name, M, N, K, flush=True)
    d = mm_inputs(K, M, N, seed=M + N)
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    out = _nan_out(M, N, gpu)
    kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    rep = mm_check(_host(out), omm.closed_form(d["lhs_T"], d["rhs"]))
    assert rep["ok"], (tc.name, rep)


def test_many_parts_deterministic_and_counters_reset(gpu):
    """Four 128x128 tiles over 64 K tiles on 256 workgroups: 64 parts per
    tile, all finishing together, so early parts and owners race to
    combine.  Twenty calls in a row give the same bits (the combiner sums in
    part order whoever it is), which also shows each call left its counters
    at zero for the next."""
    import torch

    import kernel_library as kl

    M, N, K = 256, 256, 4096
    tc = kl.TileConfig(128, 128, 64, 4, 3, variant=5)
    d = mm_inputs(K, M, N, seed=3)
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    first = _nan_out(M, N, gpu)
    kl.matmul_lhsT_rhs(a, b, cfg=tc, out=first)
    rep = mm_check(_host(first), omm.closed_form(d["lhs_T"], d["rhs"]))
    assert rep["ok"], rep
    for i in range(20):
        out = _nan_out(M, N, gpu)
        kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), first.view(torch.int16)), i


@pytest.mark.parametrize("m,name", [(16, "bm32_bn128_bk128_w4_s3_v6"), (64, "bm64_bn128_bk64_w4_s4_v6"),
                                    (128, "bm128_bn128_bk64_w4_s3_v6")])
def test_skinny_benchmark_shapes_full_output(gpu, m, name):
    """Benchmark config C5 (M x 28672 x 8192, N(0, 0.02) inputs): every output
    against a float64 product on the GPU, sampled rows against the oracle,
    and a second call bitwise equal to the first."""
    import torch

    import kernel_library as kl

    N, K = 28672, 8192
    tc = kl.TileConfig.from_name(name)
    print("stream-K C5", m, name, flush=True)
    d = mm_inputs(K, m, N, seed=0, dist=("normal", 0.02))
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    out = _nan_out(m, N, gpu)
    kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    full = _f64_check(out, a, b)
    print("all outputs vs float64:", full, flush=True)
    assert full["ok"], full
    cols = np.random.default_rng(1).integers(0, N, size=256)
    rep = mm_check(_host(out)[:, cols], omm.closed_form(d["lhs_T"], d["rhs"][:, cols]))
    assert rep["ok"], rep
    again = _nan_out(m, N, gpu)
    kl.matmul_lhsT_rhs(a, b, cfg=tc, out=again)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))


def test_two_streams_at_once(gpu):
    """Stream-K calls on two streams with no ordering between them: each
    stream has its own kept workspace, so both results are whole and
    correct."""
    import torch

    import kernel_library as kl

    tc = kl.TileConfig(64, 128, 64, 4, 4, variant=6)
    shapes = [(64, 7168, 4096), (128, 5120, 2048)]
    inputs, outs, streams = [], [], []
    for i, (M, N, K) in enumerate(shapes):
        d = mm_inputs(K, M, N, seed=30 + i)
        inputs.append((d, _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)))
        outs.append(_nan_out(M, N, gpu))
        streams.append(torch.cuda.Stream(device=gpu))
    torch.cuda.synchronize()
    for rep in range(3):
        for (d, a, b), out, st in zip(inputs, outs, streams):
            with torch.cuda.stream(st):
                kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
        torch.cuda.synchronize()
        for (d, a, b), out in zip(inputs, outs):
            rep_ = mm_check(_host(out), omm.closed_form(d["lhs_T"], d["rhs"]))
            assert rep_["ok"], (rep, rep_)
            out.fill_(float("nan"))


def test_graph_replay_matches_eager(gpu):
    """A stream-K call captured in a HIP graph takes its workspace from the
    pool, with the counters zeroed by a captured kernel; four replays with
    eager work between them each match the eager output bit for bit."""
    import torch

    import kernel_library as kl

    M, N, K = 128, 4096, 4096
    tc = kl.TileConfig(128, 128, 64, 4, 3, variant=6)
    d = mm_inputs(K, M, N, seed=7)
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    out = _nan_out(M, N, gpu)
    kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    torch.cuda.synchronize()
    eager = out.clone()
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kl.matmul_lhsT_rhs(a, b, cfg=tc, out=out)
    other = a.flip(0).contiguous()
    for rep in range(4):
        out.fill_(float("nan"))
        kl.matmul_lhsT_rhs(other, b, cfg=tc)   # eager stream-K work on the same kept workspace in between
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), rep


def test_noalloc_entry_point_matches(gpu):
    """mi_matmul_lhsT_rhs_bf16_noalloc runs the stream-K kernel with its
    workspace in the static scratch (counters zero when loaded, left zero by
    every launch): bitwise equal to the allocating entry point, twice."""
    import torch

    import kernel_library as kl
    from kernel_library import _lib

    L = _lib.lib()
    for i, (M, N, K) in enumerate([(128, 28672, 2048), (64, 4096, 8192)]):
        tc = kl.TileConfig(128 if M == 128 else 64, 128, 64, 4, 3 if M == 128 else 4, variant=6)
        d = mm_inputs(K, M, N, seed=40 + i)
        a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
        ref = kl.matmul_lhsT_rhs(a, b, cfg=tc)
        out = _nan_out(M, N, gpu)
        c = tc.to_c()
        rc = L.mi_matmul_lhsT_rhs_bf16_noalloc(a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, ctypes.byref(c),
                                               torch.cuda.current_stream(gpu).cuda_stream)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (M, N, K)
