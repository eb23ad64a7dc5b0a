"""CPU tests of the autotune runner: results table, selection, results.json,
the compile step and the pipeline's host-side checks.

The first three tests mirror the reference's only profiler-backend tests
(test/runner/test_output.py:21-56), which build ProfileResults by hand.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest

from autotune.runner import compile as rcompile
from autotune.runner.benchmark import utilisation, work_of
from autotune.runner.output import ProfileOutput, write_kernel_sources, write_results_json
from autotune.runner.types import KernelJob, ProfileResult, profiler_percent
from autotune.tune import input_specs, make_jobs
from kernel_library import _lib
from kernel_library.config import TileConfig, baseline_grid, record_tuned


def _summary_result(name: str, total_time: float, mfu: float, cfg: TileConfig | None = None) -> ProfileResult:
    summary = {"total_time": total_time, "mfu_estimated_percent": mfu, "tflops": 1.0 / total_time}
    if cfg is not None:
        summary["config"] = cfg.asdict()
    return ProfileResult(kernel_name=name, hardware_output="[128, 512] bfloat16", profiler_summary=summary)


def test_write_results_json_no_hosts_key(tmp_path):
    results = [_summary_result("k_0.hip", 0.001, 0.9)]
    write_results_json(str(tmp_path), num_kernels=1, results=results, wallclock_s=1.5)
    data = json.loads((tmp_path / "results.json").read_text())
    assert "hosts" not in data["metadata"]
    assert data["metadata"] == {"num_kernels": 1, "wallclock_s": 1.5}
    assert data["metrics"]["success"] == 1
    assert data["kernels"][0]["kernel_name"] == "k_0.hip"
    assert (tmp_path / "k_0" / "profile_summary.json").exists()


def test_write_results_json_sorts_kernels_numerically(tmp_path):
    results = [_summary_result("kernel_10.hip", 0.002, 0.5), _summary_result("kernel_2.hip", 0.001, 0.5),
               _summary_result("zeta.hip", 0.003, 0.5)]
    write_results_json(str(tmp_path), num_kernels=3, results=results, wallclock_s=1.0)
    names = [k["kernel_name"] for k in json.loads((tmp_path / "results.json").read_text())["kernels"]]
    assert names == ["kernel_2.hip", "kernel_10.hip", "zeta.hip"]


def test_profile_output_str_has_no_hosts_line():
    out = ProfileOutput(results=[_summary_result("k_0.hip", 0.001, 0.9)], compiler_logs={}, elapsed_s=2.0)
    text = str(out)
    assert "Hosts:" not in text and "Succeeded:  1/1" in text


def test_selection_metrics_and_failure_classes(tmp_path):
    fast = TileConfig(256, 128, 64, 8, 1)
    results = [
        _summary_result("a.hip", 0.003, 0.3, TileConfig(128, 128, 64, 4, 2)),
        _summary_result("b.hip", 0.001, 0.9, fast),
        ProfileResult("c.hip", "illegal config bm256_bn256_bk128_w8_s2 at M=8 N=8 K=8: [LDS over budget] LDS ..."),
        ProfileResult("d.hip", "illegal config x: [alignment] M=7"),
        ProfileResult("e.hip", "Traceback ...\nRuntimeError: hipcc failed for e.hip:\nerror: ..."),
        ProfileResult("f.hip", "Compilation timed out after 600 s"),
        ProfileResult("g.hip", "[1, 1] bfloat16", None),  # ran but produced no summary
    ]
    out = ProfileOutput(results, {}, 3.0)
    assert [s.kernel_name for s in out.successes] == ["a.hip", "b.hip"]
    assert out.best.kernel_name == "b.hip" and out.best.config == fast.name
    assert {r.kernel_name for r in out.failures} == {"c.hip", "d.hip", "e.hip", "f.hip", "g.hip"}
    text = str(out)
    assert text.index("b.hip") < text.index("a.hip")          # table sorted by time
    assert "5 failures:" in text and "Best:       0.001000 s (b.hip)" in text
    write_results_json(str(tmp_path), len(results), results, 3.0)
    m = json.loads((tmp_path / "results.json").read_text())["metrics"]
    assert m["best_kernel"] == "b.hip" and m["worst_kernel"] == "a.hip"
    assert m["best_config"] == fast.asdict()
    assert m["best_mfu"] == pytest.approx(90.0) and m["worst_mfu"] == pytest.approx(30.0)
    assert (m["success"], m["lds_over_budget"], m["illegal_config"], m["compile_error"], m["timeout"]) == (2, 1, 1, 1, 1)


def test_reference_result_fields_and_oom_metric_keys(tmp_path):
    """A caller of the reference builds ProfileResult with all six of its
    keyword arguments (reference types.py:70-98) and reads results.json's
    out-of-memory counters (output.py:225-239, :265-266): here LDS over
    budget (SBUF) and accumulator registers over budget (PSUM)."""
    full = ProfileResult(kernel_name="a.hip", hardware_output="[8, 8] bfloat16",
                         profiler_summary={"total_time": 1e-3, "mfu_estimated_percent": 0.5},
                         profile_detailed={"times_s": [1e-3]}, neff_b64="AAAA", ntff_b64="QkJC")
    assert (full.neff_b64, full.ntff_b64) == ("AAAA", "QkJC")
    bare = ProfileResult("b.hip", "[8, 8] bfloat16")
    assert bare.profiler_summary is None and bare.neff_b64 is None and bare.ntff_b64 is None
    results = [full,
               ProfileResult("c.hip", "illegal config x at M=8 N=8 K=8: [LDS over budget] LDS 262144 bytes"),
               ProfileResult("d.hip", "illegal config y at M=8 N=8 K=8: [wave tile smaller than one MFMA tile] "
                                      "each wave's accumulators exceed its share of the 512 registers"),
               ProfileResult("e.hip", "Traceback ...\nRuntimeError: boom")]
    write_results_json(str(tmp_path), len(results), results, 1.0)
    m = json.loads((tmp_path / "results.json").read_text())["metrics"]
    assert (m["success"], m["sbuf_oom"], m["psum_oom"]) == (1, 1, 1)
    for key in ("best_total_time_s", "worst_total_time_s", "best_kernel", "worst_kernel", "best_mfu", "worst_mfu",
                "best_mbu", "worst_mbu"):
        assert key in m
    # The real legality message of an over-budget wave tile carries the PSUM mark.
    import ctypes

    c = TileConfig(256, 256, 32, 1, 2, variant=1).to_c()
    rc = _lib.lib().mi_cfg_check(0, ctypes.byref(c), 512, 512, 512)
    msg = _lib.last_error()
    assert rc == _lib.MI_E_WAVE_TILE and "exceed its share of the 512 registers" in msg, (rc, msg)


def test_code_object_of_prebuilt_instances():
    """neff_b64's artifact: the gfx950 code object (an ELF) of the library's
    offload bundle that defines the instance's kernel, found by its mangled
    template name and tile parameters; None for a config the library lacks."""
    import base64

    from autotune.runner import codeobj
    from autotune.runner.benchmark import code_object_b64

    lib = str(_lib.LIB_PATH)
    seen = set()
    for fam, name in (("matmul_lhsT_rhs", "bm256_bn256_bk32_w4_s3_v1"), ("matmul_lhsT_rhs", "bm32_bn128_bk128_w4_s3_v3"),
                      ("rmsnorm_matmul", "bm128_bn512_bk32_w8_s3_v4"), ("rmsnorm_matmul", "bm256_bn256_bk32_w4_s3_v13"),
                      ("matmul_lhs_rhs", "bm128_bn128_bk64_w4_s3"), ("matmul_lhsT_rhs_f32", "bm64_bn64_bk16_w4_s1")):
        cfg = TileConfig.from_name(name)
        co = codeobj.code_object_of(lib, fam, cfg)
        assert co is not None and co[:4] == b"\x7fELF", (fam, name)
        assert codeobj.mangled_stem(fam, cfg) in co
        seen.add(hash(co))
        assert base64.b64decode(code_object_b64(lib, fam, cfg)) == co
    assert len(seen) >= 4                      # different translation units, different code objects
    assert codeobj.code_object_of(lib, "matmul_lhsT_rhs", TileConfig(512, 512, 32, 4, 3, variant=1)) is None
    assert codeobj.mangled_stem("matmul_lhsT_rhs", TileConfig(256, 256, 32, 4, 3, variant=1)) == \
        b"28mm_lhsT_rhs_bf16_pipe_kernelILi256ELi256ELi32ELi4ELi3E"


def test_profiler_percent_contract():
    assert profiler_percent({"x": 0.5}, "x") == 50.0
    assert profiler_percent({"x": -1.0}, "x") is None       # negative sentinel
    assert profiler_percent({}, "x") is None and profiler_percent(None, "x") is None


def test_work_and_utilisation_known_answers():
    flops, nbytes = work_of("matmul_lhsT_rhs", 8192, 8192, 8192, "bfloat16")
    assert flops == 2 * 8192**3 and nbytes == 3 * 8192 * 8192 * 2
    f2, b2 = work_of("rmsnorm_matmul", 4096, 4096, 4096, "bfloat16", has_gamma=True)
    assert b2 == 3 * 4096 * 4096 * 2 + 4096 * 2
    u = utilisation(flops, nbytes, 1e-3, "bfloat16")
    assert u["tflops"] == pytest.approx(1099.511627776)
    assert u["mfu_estimated_percent"] == pytest.approx(1099.511627776 / 2500)
    assert u["mbu_estimated_percent"] == pytest.approx(402.653184 / 8000)
    assert u["mfu_max_achievable_estimated_percent"] == 1.0
    skinny = utilisation(*work_of("matmul_lhsT_rhs", 16, 28672, 8192, "bfloat16"), 1e-4, "bfloat16")
    assert skinny["mfu_max_achievable_estimated_percent"] < 0.06   # HBM-bound shape


def test_render_parse_roundtrip_and_aliases():
    for fam in ("matmul_lhsT_rhs", "rmsnorm_matmul", "matmul_lhsT_rhs_nkigym", "rmsnorm_matmul_online",
                "matmul_lhs_rhs", "matmul_lhs_rhs_nkigym"):
        cfg = TileConfig(128, 256, 64, 8, 2, variant=1 if "rms" in fam else 0)
        src = rcompile.render_source(fam, cfg)
        got_fam, got_cfg = rcompile.parse_source(src)
        assert got_fam == rcompile.canonical_name(fam) and got_cfg == cfg
        assert "#include \"mi_registry.hpp\"" in src
    with pytest.raises(ValueError):
        rcompile.parse_source("__global__ void k() {}")
    assert rcompile.problem_shape("matmul_lhsT_rhs", input_specs("matmul_lhsT_rhs", 64, 96, 128)) == (64, 96, 128)
    assert rcompile.problem_shape("rmsnorm_matmul", input_specs("rmsnorm_matmul", 64, 96, 128)) == (64, 96, 128)
    assert rcompile.problem_shape("matmul_lhs_rhs", input_specs("matmul_lhs_rhs", 64, 96, 128)) == (64, 96, 128)


@pytest.mark.parametrize("fam,variants", [("matmul_lhsT_rhs", (0, 1, 2, 3, 4, 5, 6)), ("matmul_lhs_rhs", (0, 1, 2)),
                                          ("rmsnorm_matmul", (0, 1, 4, 5, 11, 12, 13, 14, 15, 16))])
def test_jit_units_instantiate_every_variant(fam, variants, tmp_path):
    """The generated single-config unit of every variant names a real template
    and table row: hipcc parses and instantiates it (device side, no codegen),
    and the row carries the config's variant."""
    import shutil
    import subprocess

    import build_lib

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    from kernel_library.config import compiled_configs

    prebuilt = compiled_configs(fam)
    for v in variants:
        cfg = next(c for c in prebuilt if c.variant == v)   # a config the template is known to take
        src = rcompile.render_source(fam, cfg)
        assert "prebuilt-only" not in src, (fam, v)
        unit = tmp_path / f"{fam}_{v}.hip"
        unit.write_text(src)
        flags = [f for f in build_lib.HIPCC_FLAGS if f != "-fPIC"]
        proc = subprocess.run([hipcc, *flags, f"-I{build_lib.CSRC}", f"-I{build_lib.INCLUDE}", "--cuda-device-only",
                               "-fsyntax-only", str(unit)], capture_output=True, text=True)
        assert proc.returncode == 0, (fam, v, proc.stderr[-2000:])
    # a variant without a template is reported, not guessed
    assert "prebuilt-only" in rcompile.render_source("matmul_lhs_rhs", TileConfig(128, 256, 32, 4, 2, variant=3))


def test_compile_one_prebuilt_and_rejections(tmp_path):
    specs = input_specs("matmul_lhsT_rhs", 1024, 1024, 1024)
    src = rcompile.render_source("matmul_lhsT_rhs", TileConfig(256, 128, 64, 8, 1))
    cr = rcompile.compile_one("a.hip", src, "matmul_lhsT_rhs", specs, str(tmp_path))
    assert cr.error == "" and cr.library_path == str(_lib.LIB_PATH)
    big = rcompile.render_source("matmul_lhsT_rhs", TileConfig(256, 256, 128, 8, 2))
    cr = rcompile.compile_one("b.hip", big, "matmul_lhsT_rhs", specs, str(tmp_path))
    assert "LDS over budget" in cr.error and cr.library_path == ""
    cr = rcompile.compile_one("c.hip", src, "rmsnorm_matmul", specs, str(tmp_path))
    assert "does not match" in cr.error
    cr = rcompile.compile_one("d.hip", "garbage", "matmul_lhsT_rhs", specs, str(tmp_path))
    assert "Traceback" in cr.error
    jit = rcompile.render_source("matmul_lhsT_rhs", TileConfig(512, 128, 32, 8, 1))
    cr = rcompile.compile_one("e.hip", jit, "matmul_lhsT_rhs", specs, str(tmp_path), allow_jit=False)
    assert "JIT is off" in cr.error


def test_compile_one_builds_a_non_prebuilt_instance(tmp_path):
    """A legal config outside the prebuilt table is built by hipcc into a library with the full C ABI."""
    specs = input_specs("matmul_lhsT_rhs", 1024, 1024, 1024)
    cfg = TileConfig(512, 128, 32, 8, 1)
    cr = rcompile.compile_one("jit_0.hip", rcompile.render_source("matmul_lhsT_rhs", cfg), "matmul_lhsT_rhs", specs,
                              str(tmp_path))
    assert cr.error == "", cr.error
    lib = _lib.load(cr.library_path)
    assert lib.mi_num_configs(_lib.MI_KERNEL_MATMUL_LHST_RHS_BF16) == 1
    c = cfg.to_c()
    import ctypes

    assert lib.mi_cfg_check(_lib.MI_KERNEL_MATMUL_LHST_RHS_BF16, ctypes.byref(c), 1024, 1024, 1024) == 0
    assert lib.mi_num_configs(_lib.MI_KERNEL_RMSNORM_MATMUL_BF16) == 0


def test_compile_timeout_is_an_error_string(tmp_path):
    specs = input_specs("matmul_lhsT_rhs", 1024, 1024, 1024)
    src = rcompile.render_source("matmul_lhsT_rhs", TileConfig(512, 128, 64, 8, 1))
    cr = rcompile.compile_one("slow.hip", src, "matmul_lhsT_rhs", specs, str(tmp_path), timeout_s=0.01)
    assert cr.error.startswith("Compilation timed out")


def test_pipeline_rejects_more_than_one_device(tmp_path):
    from autotune.runner.driver import run_pipeline

    job = next(iter(make_jobs("matmul_lhsT_rhs", 256, 256, 256, [TileConfig(128, 128, 64, 4, 2)]).values()))
    with pytest.raises(RuntimeError, match="one GPU"):
        run_pipeline({"k.hip": job._replace(lnc=2)}, 0, False, False, work_dir=str(tmp_path / "w"))


def test_profile_requires_a_gfx950_device(tmp_path):
    """Environment faults raise (reference detect.py:13-19); on this CPU host no HIP device is visible."""
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from autotune.runner.api import profile

    jobs = make_jobs("matmul_lhsT_rhs", 256, 256, 256, [TileConfig(128, 128, 64, 4, 2)])
    with pytest.raises(RuntimeError, match="HIP device"):
        profile(jobs, str(tmp_path / "cache"), 0)
    with pytest.raises(ValueError):
        profile(jobs, "", 0, neuron_platform_target="sm_90")


def test_profile_takes_the_reference_call(tmp_path, monkeypatch):
    """The reference's drivers call ``profile(jobs, cache_dir=..., seed=...,
    neuron_platform_target=..., collect_detailed_profile=...)`` with jobs
    built as ``KernelJob(..., neuronx_cc_args=...)``
    (examples/tune_matmul_lhsT_rhs.py:259-265; examples/profile_hand_90mfu.py:
    101-111): the same call, word for word, runs here.  The pipeline is
    replaced by a recorder (no GPU on this host)."""
    from autotune.runner import api
    from autotune.runner.output import ProfileOutput

    seen = {}

    def recorder(kernels, **kw):
        seen.update(kw, kernels=kernels)
        return [], {}

    monkeypatch.setattr(api, "run_pipeline", recorder)
    M = N = K = 2048
    input_specs_ref = {"lhs_T": ((K, M), "bfloat16"), "rhs": ((K, N), "bfloat16")}
    neuronx_cc_args = ("enable-linear-scan-allocation=false", "enable-instruction-scheduling=false")
    jobs = {
        "hand_90mfu": KernelJob(
            source=rcompile.render_source("matmul_lhsT_rhs_nkigym", TileConfig(256, 256, 32, 4, 3, variant=1)),
            func_name="matmul_lhsT_rhs_nkigym",
            output_shape=(M, N),
            input_specs=input_specs_ref,
            neuronx_cc_args=neuronx_cc_args,
        )
    }
    cache_dir = str(tmp_path / "profile_hand_90mfu")
    output = api.profile(
        jobs,
        cache_dir=cache_dir,
        seed=0,
        neuron_platform_target="trn2",
        collect_detailed_profile=False,
    )
    assert isinstance(output, ProfileOutput) and output.results == [] and output.cache_dir == cache_dir
    assert seen["kernels"] is jobs and seen["seed"] == 0 and seen["collect_detailed_profile"] is False
    job = jobs["hand_90mfu"]
    assert job.hipcc_args == () and job.ignored_args == neuronx_cc_args     # Neuron options: not hipcc flags
    assert KernelJob(job.source, job.func_name, (M, N), input_specs_ref, ("-DX=1", "opt=1")).hipcc_args == ("-DX=1",)
    assert (tmp_path / "profile_hand_90mfu" / "hand_90mfu" / "hand_90mfu.hip").exists()
    assert api.resolve_target("gfx950") == api.resolve_target("trn2") == "gfx950"


def test_make_jobs_and_cache_sources(tmp_path):
    cfgs = [TileConfig(128, 128, 64, 4, 2), TileConfig(256, 128, 64, 8, 1)]
    jobs = make_jobs("rmsnorm_matmul", 4096, 4096, 4096, cfgs)
    assert list(jobs) == [c.name + ".hip" for c in cfgs]
    job = jobs[cfgs[0].name + ".hip"]
    assert isinstance(job, KernelJob) and job.output_shape == (4096, 4096)
    assert list(job.input_specs) == ["lhs", "gamma", "rhs"]
    assert job.input_dists["rhs"] == ("normal", 1 / 64)
    write_kernel_sources(str(tmp_path), jobs)
    text = (tmp_path / cfgs[1].name / (cfgs[1].name + ".hip")).read_text()
    assert rcompile.parse_source(text)[1] == cfgs[1]


def test_baseline_grid_and_tuned_table(tmp_path):
    grid = baseline_grid()
    assert len(grid) == 72 and len(set(grid)) == 72
    assert len(baseline_grid((0, 1))) == 144
    path = tmp_path / "tuned.json"
    record_tuned("matmul_lhsT_rhs", 64, 64, 64, grid[5], path=path, extra={"tflops": 1.0})
    record_tuned("rmsnorm_matmul", 64, 64, 64, grid[6], path=path)
    doc = json.loads(path.read_text())
    assert doc["configs"]["matmul_lhsT_rhs:64x64x64"] == grid[5].asdict()
    assert doc["measurements"]["matmul_lhsT_rhs:64x64x64"] == {"tflops": 1.0}
    assert TileConfig(**doc["configs"]["rmsnorm_matmul:64x64x64"]) == grid[6]


def test_detailed_profile_trace_helpers(tmp_path, monkeypatch):
    """Replay job round trip, the profiler command shape, stats parsing, and
    a missing profiler reported as data (never raised)."""
    import autotune.runner.trace as tr
    from autotune.runner.replay import main as replay_main

    specs = input_specs("matmul_lhsT_rhs", 64, 96, 128)
    path = tr.write_replay_job(str(tmp_path / "k0"), "k0.hip", "matmul_lhsT_rhs", "/x/lib.so",
                               TileConfig(128, 128, 64, 4, 2).asdict(), (64, 96, 128), specs,
                               {"lhs_T": ("normal", 0.02)}, 7, 3, 5)
    job = json.loads(Path(path).read_text())
    assert job["shape"] == [64, 96, 128] and job["input_specs"]["lhs_T"] == [[128, 64], "bfloat16"]
    assert job["input_dists"] == {"lhs_T": ["normal", 0.02]} and job["seed"] == 7
    cmd = tr.rocprof_command(str(tmp_path / "out"), path)
    i = cmd.index("--")
    assert "--kernel-trace" in cmd[:i] and "--pmc" not in cmd
    assert cmd[i + 1:i + 4] == [cmd[i + 1], "-u", "-m"] and cmd[i + 4] == "autotune.runner.replay"
    csv_path = tmp_path / "stats.csv"
    csv_path.write_text('"Name","Calls","TotalDurationNs","AverageNs","Percentage","MinNs","MaxNs","StdDev"\n'
                        '"void at::native::copy(int)",2,100,50.0,1.0,40,60,1.0\n'
                        '"void mi::mm_lhsT_rhs_bf16_pipe_kernel<256, 256, 32, 4, 3>(int)",110,85577516,777977.4,'
                        '99.8,742629,1029515,52412.2\n')
    row = tr.parse_kernel_stats(str(csv_path))
    assert row["calls"] == 110 and row["avg_ns"] == 777977.4 and "pipe_kernel" in row["kernel"]
    assert len(row["kernels"]) == 1
    with open(csv_path, "a") as f:   # a split-K config: the main kernel and its summing kernel
        f.write('"void mi::splitk_sum_kernel<0>(float const*)",110,1100000,10000.0,0.2,9000,12000,100.0\n')
    row = tr.parse_kernel_stats(str(csv_path))
    assert "pipe_kernel" in row["kernel"] and [r["calls"] for r in row["kernels"]] == [110, 110]
    monkeypatch.setattr(tr.shutil, "which", lambda name: None)
    assert "not found" in tr.trace_kernel(str(tmp_path / "k0"), path)["error"]
    with pytest.raises(SystemExit):          # usage error: no replay file
        replay_main([])


def test_tune_cli_named_configs_and_detailed_needs_cache(monkeypatch):
    """--configs names the configs to time (split_k included); --detailed without --cache is a usage error."""
    from autotune import tune as tmod

    seen = {}

    def fake_tune(fam, M, N, K, configs, *a, **kw):
        seen.update(fam=fam, shape=(M, N, K), configs=configs, detailed=kw.get("detailed"),
                    with_gamma=kw.get("with_gamma"))
        return tmod.TuneResult(None, None, "", None)

    monkeypatch.setattr(tmod, "tune", fake_tune)
    rc = tmod.main(["--kernel", "matmul_lhsT_rhs", "--shape", "512", "512", "32768", "--configs",
                    "bm64_bn64_bk64_w4_s4_v1,bm64_bn64_bk64_w4_s4_v1_k4"])
    assert rc == 1 and seen["shape"] == (512, 512, 32768) and seen["detailed"] is False
    assert [c.split_k for c in seen["configs"]] == [1, 4]
    with pytest.raises(SystemExit):
        tmod.main(["--configs", "bm64_bn64_bk64_w4_s4_v1", "--detailed"])
    # rmsnorm_matmul_online is the reference's no-gamma contract
    tmod.main(["--kernel", "rmsnorm_matmul_online", "--shape", "256", "256", "512"])
    assert seen["fam"] == "rmsnorm_matmul" and seen["with_gamma"] is False
    tmod.main(["--kernel", "rmsnorm_matmul", "--shape", "256", "256", "512"])
    assert seen["with_gamma"] is True


def test_tune_cli_clears_only_a_tune_cache(monkeypatch, tmp_path):
    """--cache is cleared before the sweep, but a non-empty directory without results.json is refused untouched."""
    from autotune import tune as tmod

    monkeypatch.setattr(tmod, "tune", lambda *a, **kw: tmod.TuneResult(None, None, "", None))
    other = tmp_path / "home"
    other.mkdir()
    (other / "notes.txt").write_text("keep me")
    with pytest.raises(SystemExit):
        tmod.main(["--configs", "bm64_bn64_bk64_w4_s4_v1", "--cache", str(other)])
    assert (other / "notes.txt").read_text() == "keep me"
    old = tmp_path / "cache"
    old.mkdir()
    (old / "results.json").write_text("{}")
    (old / "stale.hip").write_text("")
    tmod.main(["--configs", "bm64_bn64_bk64_w4_s4_v1", "--cache", str(old)])
    assert old.is_dir() and not any(old.iterdir())
    fresh = tmp_path / "new" / "cache"
    tmod.main(["--configs", "bm64_bn64_bk64_w4_s4_v1", "--cache", str(fresh)])
    assert fresh.is_dir()


def test_baseline_row_numerics_failures_and_counters(tmp_path):
    """The results model renders the vendor baseline row and the measured
    counters in the table and results.json, and a numerics failure is a
    failure row, never a selectable success."""
    from autotune.runner.output import ResultsModel, natural_key

    fast, slow = TileConfig(256, 256, 32, 4, 3, variant=1), TileConfig(128, 128, 64, 4, 2, variant=1)
    a = _summary_result("fast.hip", 0.0010, 0.6, fast)
    a = a._replace(profile_detailed={"counters": {"mfma_busy_percent": 87.5, "hbm_gbps": 2100.0,
                                                  "engine_clock_mhz": 1620.0}})
    b = _summary_result("slow.hip", 0.0020, 0.3, slow)
    wrong = ProfileResult("wrong.hip", "numerics check failed: max_abs 3.2, max_rel 0.8 (atol 0.005, rtol 0.01), 0 "
                                       "non-finite values")
    base = ProfileResult("vendor_matmul_lhsT_rhs", "[256, 256] bfloat16",
                         {"total_time": 0.0015, "mfu_estimated_percent": 0.4, "tflops": 1.0,
                          "library": "torch.matmul (hipBLASLt)"})
    out = ProfileOutput([a, b, wrong], {}, 1.0, baseline=base)
    assert out.best.kernel_name == "fast.hip" and len(out.successes) == 2
    assert [r.kernel_name for r in out.failures] == ["wrong.hip"]
    text = str(out)
    assert "vendor_matmul_lhsT_rhs" in text and "1.500x faster" in text
    assert "87.5%" in text and "1620" in text
    write_results_json(str(tmp_path), 3, out.results, 1.0, base)
    doc = json.loads((tmp_path / "results.json").read_text())
    assert doc["metrics"]["numerics_mismatch"] == 1 and doc["metrics"]["success"] == 2
    assert doc["metrics"]["best_speedup_vs_baseline"] == pytest.approx(1.5)
    assert doc["baseline"]["library"] == "torch.matmul (hipBLASLt)"
    row = next(k for k in doc["kernels"] if k["kernel_name"] == "fast.hip")
    assert row["mfma_busy_percent"] == 87.5 and row["engine_clock_mhz"] == 1620.0
    assert (tmp_path / "vendor_matmul_lhsT_rhs" / "profile_summary.json").exists()
    # natural order: digit runs by value
    names = ["k_10", "k_2", "bm256_x", "bm64_x"]
    assert sorted(names, key=natural_key) == ["bm64_x", "bm256_x", "k_2", "k_10"]
    assert ResultsModel.of([]).fastest() is None


def test_counter_parsing_and_derivation(tmp_path):
    """Counter passes -> per-call figures: calls grouped over the instance's
    kernels (a split call has two), the warm-up call dropped, the median
    call kept, byte counters scaled by the device copy before the first
    kernel, MFMA busy = busy cycles per SIMD over active cycles per XCD,
    clock = active cycles per XCD over the call's duration."""
    from autotune.runner.trace import CALIBRATE_MIB, derive, per_call_counters, read_counter_csv

    def csv_of(rows):
        head = '"Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value","Start_Timestamp","End_Timestamp"\n'
        return head + "".join(f'{i},"{n}","{c}",{v},{s},{e}\n' for i, n, c, v, s, e in rows)

    cal = CALIBRATE_MIB << 20
    rows = [(1, "__amd_rocclr_copyBuffer", "FETCH_SIZE", cal / 1024 / 2, 0, 100)]   # reads count half
    t = 1000
    for call in range(4):                      # warm-up + 3 timed calls, 2 kernels each
        ns = (1000, 3000, 2000, 2500)[call]
        for k, frac in (("mi::main_kernel<1>(int)", 0.75), ("mi::sum_kernel<0>(float)", 0.25)):
            d = 2 + 2 * call + (k.startswith("mi::sum"))
            dur = int(ns * frac)
            rows += [(d, k, "GRBM_GUI_ACTIVE", 8 * 1.6 * dur, t, t + dur),
                     (d, k, "SQ_VALU_MFMA_BUSY_CYCLES", 1024 * 0.8 * 1.6 * dur if "main" in k else 0, t, t + dur),
                     (d, k, "FETCH_SIZE", 1000.0, t, t + dur)]
            t += dur + 10
    p = tmp_path / "c.csv"
    p.write_text(csv_of(rows))
    pc = per_call_counters(read_counter_csv(str(p)), calls=4, calibrate_bytes=cal)
    assert pc["ns"] == 2500 and pc["scale"]["FETCH_SIZE"] == pytest.approx(2.0)
    assert pc["counters"]["FETCH_SIZE"] == 2000.0 and len(pc["kernels"]) == 2
    pc2 = {**pc, "counters": {"WRITE_SIZE": 500.0}, "scale": {"WRITE_SIZE": 1.0}}
    short = derive([pc, pc2])
    assert "engine_clock_mhz" not in short and "note" in short and short["hbm_gbps"] > 0   # a 2.5 us call
    pc = {**pc, "ns": pc["ns"] * 40, "counters": {k: v * 40 for k, v in pc["counters"].items()}}
    pc2 = {**pc2, "ns": pc["ns"]}
    d = derive([pc, pc2])
    assert d["engine_clock_mhz"] == pytest.approx(1600.0)
    assert d["mfma_busy_percent"] == pytest.approx(80.0 * 0.75)
    assert d["hbm_bytes"] == pytest.approx(40 * 2000 * 1024 * 2.0 + 500 * 1024)
    assert d["hbm_gbps"] == pytest.approx(d["hbm_bytes"] / pc["ns"])
    with pytest.raises(ValueError):
        per_call_counters(read_counter_csv(str(p)), calls=3, calibrate_bytes=cal)
