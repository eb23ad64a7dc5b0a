"""ctypes binding of libmi_probe.so: the measurement probes bench.py reports.

Not part of the kernel_library API (nothing on the kernel path calls it):

* :func:`clocked_lhsT_rhs` runs the clocked twin of the pipelined lhsT.rhs
  kernel -- the shipped kernel plus two counter reads per workgroup -- and
  returns the engine clock it ran at (engine cycles over 100 MHz real-time
  ticks, summed over workgroups) and its launch time;
* :func:`mfma_ceiling` runs the MFMA work of a 128x128 wave tile on every
  SIMD with operands from registers (mode 0) or read from LDS the way the
  kernel reads them (mode 1), without global memory traffic, and returns
  its rate and clock;
* :func:`panel_stream` runs the kernels' LDS-direct K-panel loads alone
  (one workgroup per CU, no LDS reads, no MFMA) over a buffer region and
  returns the rate they reach: from L2 when the region fits in it.
"""

from __future__ import annotations

import ctypes
import statistics
from pathlib import Path

from kernel_library import _lib

PROBE_PATH = Path(__file__).resolve().parent / "libmi_probe.so"
PEAK_BF16_TFLOPS = 2500.0
PEAK_CLOCK_MHZ = 2400.0
_HANDLE: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load libmi_probe.so once; ImportError if it was never built."""
    global _HANDLE
    if _HANDLE is None:
        if not PROBE_PATH.exists():
            raise ImportError(f"{PROBE_PATH} not found: build it with `python nki-autotune_amd/build_lib.py`")
        h = ctypes.CDLL(str(PROBE_PATH))
        vp, ci = ctypes.c_void_p, ctypes.c_int
        h.mi_probe_clocked_lhsT_rhs.restype = ci
        h.mi_probe_clocked_lhsT_rhs.argtypes = [vp, vp, vp, ci, ci, ci, ctypes.POINTER(_lib.MiTileCfg), vp, vp]
        h.mi_probe_mfma.restype = ci
        h.mi_probe_mfma.argtypes = [vp, ctypes.c_longlong, vp, vp, ci, ci, vp]
        h.mi_probe_panel_stream.restype = ci
        h.mi_probe_panel_stream.argtypes = [vp, ctypes.c_ulonglong, ci, ctypes.c_ulonglong, ci, ci, ci, ci, vp, vp]
        _HANDLE = h
    return _HANDLE


def _clock_mhz(clk) -> float:
    """Engine clock from per-workgroup (cycles, 100 MHz ticks) pairs: sum of cycles per microsecond."""
    c = clk.view(-1, 2).double().sum(dim=0)
    return float(c[0] / (c[1] / 100.0))


def clocked_lhsT_rhs(lhs_T, rhs, out, cfg, launches: int = 20, warmup: int = 5) -> dict | None:
    """Clock and launch time of the pipelined lhsT.rhs kernel at ``cfg``, or None if it has no clocked twin."""
    import torch

    K, M = lhs_T.shape
    N = rhs.shape[1]
    grid = -(-M // cfg.block_m) * -(-N // cfg.block_n)
    clk = torch.zeros((launches + warmup, grid, 2), dtype=torch.int64, device=lhs_T.device)
    c = cfg.to_c()
    stream = torch.cuda.current_stream(lhs_T.device)
    events = []
    for i in range(launches + warmup):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        rc = lib().mi_probe_clocked_lhsT_rhs(lhs_T.data_ptr(), rhs.data_ptr(), out.data_ptr(), M, N, K,
                                            ctypes.byref(c), clk[i].data_ptr(), stream.cuda_stream)
        e1.record(stream)
        if rc == _lib.MI_E_NO_INSTANCE:
            return None
        if rc != 0:
            raise _lib.KernelLibraryError(rc, f"clocked twin of {cfg.name} failed")
        events.append((e0, e1))
    torch.cuda.synchronize()
    mhz = [_clock_mhz(clk[i]) for i in range(warmup, launches + warmup)]
    us = [events[i][0].elapsed_time(events[i][1]) * 1e3 for i in range(warmup, launches + warmup)]
    return {"clock_mhz": round(statistics.median(mhz), 1), "us": round(statistics.median(us), 1),
            "launches": launches}


def mfma_ceiling(src, mode: int, iters: int = 512, launches: int = 10, warmup: int = 3) -> dict:
    """Rate and clock of the MFMA probe (mode 0 registers, 1 LDS reads) on operands drawn from ``src`` (bf16)."""
    import torch

    out = torch.empty(65536, dtype=torch.float32, device=src.device)
    clk = torch.zeros((launches + warmup, 256, 2), dtype=torch.int64, device=src.device)
    stream = torch.cuda.current_stream(src.device)
    events = []
    for i in range(launches + warmup):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        rc = lib().mi_probe_mfma(src.data_ptr(), src.numel(), out.data_ptr(), clk[i].data_ptr(), iters, mode,
                                 stream.cuda_stream)
        e1.record(stream)
        if rc != 0:
            raise _lib.KernelLibraryError(rc, "MFMA probe failed")
        events.append((e0, e1))
    torch.cuda.synchronize()
    flop = 1024 * iters * 64 * 2.0 * 32 * 32 * 16
    us = statistics.median(events[i][0].elapsed_time(events[i][1]) * 1e3 for i in range(warmup, launches + warmup))
    mhz = statistics.median(_clock_mhz(clk[i]) for i in range(warmup, launches + warmup))
    tf = flop / (us * 1e-6) / 1e12
    return {"tflops": round(tf, 1), "pct_mfma_peak": round(100 * tf / PEAK_BF16_TFLOPS, 1),
            "clock_mhz": round(mhz, 1),
            "pct_of_peak_at_that_clock": round(100 * tf / (PEAK_BF16_TFLOPS * mhz / PEAK_CLOCK_MHZ), 1)}


def panel_stream(buf, region: int, waves: int, inflight: int, rounds: int, row_bytes: int = 1024,
                 pitch: int = 1024, wgs: int = 256, launches: int = 10, warmup: int = 3) -> dict:
    """Rate of the LDS-direct panel loads alone over ``buf``'s first ``region`` bytes.

    ``buf`` is read as a matrix of ``pitch``-byte rows, each panel load
    taking ``row_bytes`` of 1024 / row_bytes consecutive rows (the K panel
    of an MN-contiguous operand whose rows are ``pitch`` bytes); the default
    reads consecutive 1 KiB chunks.  ``wgs`` workgroups (one per CU) of
    ``waves`` waves, each wave keeping ``inflight`` 1 KiB loads in flight
    for ``rounds * inflight`` loads.
    Returns the median launch time, the aggregate GB/s, the engine clock,
    bytes per clock per CU and 128-byte L2 requests per clock per XCD.
    """
    import torch

    # The kernel's buffer descriptor spans `region` bytes from buf's start,
    # so every load stays inside buf only if region fits in it.
    if not buf.is_contiguous():
        raise ValueError("panel_stream needs a contiguous buffer")
    if region <= 0 or region > buf.numel() * buf.element_size():
        raise ValueError(f"region of {region} bytes is outside the {buf.numel() * buf.element_size()}-byte buffer")
    clk = torch.zeros((launches + warmup, wgs, 2), dtype=torch.int64, device=buf.device)
    stream = torch.cuda.current_stream(buf.device)
    events = []
    for i in range(launches + warmup):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        rc = lib().mi_probe_panel_stream(buf.data_ptr(), region, row_bytes, pitch, waves, inflight, wgs, rounds,
                                         clk[i].data_ptr(), stream.cuda_stream)
        e1.record(stream)
        if rc != 0:
            raise _lib.KernelLibraryError(rc, f"panel stream probe w{waves} inflight {inflight} failed")
        events.append((e0, e1))
    torch.cuda.synchronize()
    nbytes = float(wgs) * waves * rounds * inflight * 1024
    us = statistics.median(events[i][0].elapsed_time(events[i][1]) * 1e3 for i in range(warmup, launches + warmup))
    mhz = statistics.median(_clock_mhz(clk[i]) for i in range(warmup, launches + warmup))
    cycles = us * mhz
    return {"waves": waves, "inflight": inflight, "row_bytes": row_bytes, "pitch": pitch,
            "region_mib": round(region / 2 ** 20, 2), "us": round(us, 1),
            "gbs": round(nbytes / (us * 1e-6) / 1e9, 1), "clock_mhz": round(mhz, 1),
            "bytes_per_clk_per_cu": round(nbytes / wgs / cycles, 1),
            "l2_req_per_clk_per_xcd": round(nbytes / 128 / 8 / cycles, 2)}


__all__ = ["clocked_lhsT_rhs", "lib", "mfma_ceiling", "panel_stream", "PROBE_PATH"]
