"""mi_matmul_lhsT_rhs_bf16_noalloc (C ABI) against mi_matmul_lhsT_rhs_bf16.

The no-alloc entry point runs the same kernels with its split-K workspace in
a static device array instead of a pool allocation, so on the same inputs
and config its output must equal the allocating entry point's bit for bit.
Two calls in a row (the second smaller, reusing the scratch the first one
filled), an unsplit config, the rejection of a config whose workspace
exceeds the scratch, and the absence of any allocation once the scratch is
resident.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from helpers import mm_check, mm_inputs
from oracle import matmul as omm

pytestmark = pytest.mark.gpu


def _dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(device)


def _call(fn, a, b, out, M, N, K, cfg):
    import torch

    from kernel_library import _lib

    c = cfg.to_c()
    rc = fn(a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, ctypes.byref(c),
            torch.cuda.current_stream(a.device).cuda_stream)
    return rc, _lib.last_error()


def test_noalloc_matches_allocating_entry_point(gpu):
    import torch

    import kernel_library as kl
    from kernel_library import _lib

    L = _lib.lib()
    cases = [
        # (M, N, K, config): split-K first (4 MiB of workspace), then a smaller
        # split-K call on the same scratch, then an unsplit config.
        (512, 512, 32768, kl.TileConfig.from_name("bm64_bn64_bk64_w4_s4_v1_k4")),
        (256, 384, 8192, kl.TileConfig.from_name("bm64_bn64_bk64_w4_s4_v1_k2")),
        (1024, 1024, 1024, kl.TileConfig.from_name("bm256_bn256_bk32_w4_s3_v1")),
    ]
    for i, (M, N, K, cfg) in enumerate(cases):
        print(f"no-alloc case {i}: M={M} N={N} K={K} {cfg.name}", flush=True)
        d = mm_inputs(K, M, N, seed=20 + i)
        a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
        ref = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        rc, msg = _call(L.mi_matmul_lhsT_rhs_bf16, a, b, ref, M, N, K, cfg)
        assert rc == 0, msg
        rc, msg = _call(L.mi_matmul_lhsT_rhs_bf16_noalloc, a, b, got, M, N, K, cfg)
        assert rc == 0, msg
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, N, K, cfg.name)
        rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(i).integers(0, M, size=16)]))
        host = got.float().cpu().numpy()
        rep = mm_check(host[rows], omm.closed_form(d["lhs_T"][:, rows], d["rhs"]))
        assert rep["ok"], (cfg.name, rep)


def test_noalloc_allocates_nothing_and_rejects_oversize(gpu):
    import torch

    import kernel_library as kl
    from kernel_library import _lib

    L = _lib.lib()
    M, N, K = 512, 1024, 16384
    cfg = kl.TileConfig.from_name("bm64_bn64_bk64_w4_s4_v1_k8")   # 16 MiB of partial products
    d = mm_inputs(K, M, N, seed=31)
    a, b = _dev(d["lhs_T"], gpu), _dev(d["rhs"], gpu)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    rc, msg = _call(L.mi_matmul_lhsT_rhs_bf16_noalloc, a, b, out, M, N, K, cfg)   # scratch resident from here
    assert rc == 0, msg
    torch.cuda.synchronize()
    first = out.clone()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(gpu)[0]
    for _ in range(5):
        rc, msg = _call(L.mi_matmul_lhsT_rhs_bf16_noalloc, a, b, out, M, N, K, cfg)
        assert rc == 0, msg
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(gpu)[0] >= free0
    assert torch.equal(out, first)
    # 4 x 4096 x 4096 x 4 bytes = 256 MiB of partial products: over the scratch, rejected before any launch.
    big = kl.TileConfig.from_name("bm256_bn256_bk32_w4_s3_v1_k4")
    a2 = torch.zeros((8192, 4096), dtype=torch.bfloat16, device=gpu)
    b2 = torch.zeros((8192, 4096), dtype=torch.bfloat16, device=gpu)
    o2 = torch.empty((4096, 4096), dtype=torch.bfloat16, device=gpu)
    rc, msg = _call(L.mi_matmul_lhsT_rhs_bf16_noalloc, a2, b2, o2, 4096, 4096, 8192, big)
    assert rc == _lib.MI_E_RANGE and "static scratch" in msg, (rc, msg)
    assert _lib.NOALLOC_SCRATCH_BYTES < 4 * 4096 * 4096 * 4
