"""bench.py's command-line contract, on the CPU: it measures one GPU only, so --gpus above 1 (or a
WORLD_SIZE above 1 from a distributed launcher) exits with status 2 and a message before anything
touches a device; the module itself imports without side effects."""
import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, BENCH] + args, cwd=ROOT, env=env,
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run(["--gpus", "8"])
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_distributed_launch_exits_with_a_message():
    r = _run(["--gpus", "1"], {"WORLD_SIZE": "2"})
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_module_imports_without_running():
    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert callable(mod.main)
    assert mod.PEAK_GBS == 8000.0


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


KERNEL_LINES = [  # (name, configuration) of every line the suite measures
    ("residual_layernorm_f32_256x512", 1), ("embed_pe_prefill_1024x512", 2),
    ("embed_pe_hot_row_ceiling_1024x512", 2), ("embed_pe_prefill_pos0_511_2x512x512", 2),
    ("t2s_prefill_input_pos0_511_2x512x512", 2), ("embed_pe_prefill_distinct_pos_2x512x512", 2),
    ("embed_pe_decode_64x512", 2),
    ("embed_pe_text_rows_512x512", 2), ("residual_layernorm_f16_64x512", 2),
    ("bias_relu_f16_64x2048", 2), ("bias_gelu_f16_512x4096", 3),
    ("residual_layernorm_f16_512x1024_eps1e-12", 3), ("groupnorm_gelu_f32_512x31999", 4),
    ("residual_layernorm_f16_499x768", 4), ("bias_gelu_f16_499x3072", 4)] + [
    (f"sovits_{k}_{d}_24x320000", 5) for k in ("K3", "K2", "K1") for d in ("f32", "f16")] + [
    (f"gemv_{n}", 2) for n in ("qkv_bias_f32out_64x1536x512", "outproj_bias_residual_64x512x512",
                               "w1_bias_relu_64x2048x512", "w2_bias_residual_64x512x2048",
                               "logits_f32out_64x1025x512", "read_dominated_16x2048x512")] + [
    ("decode_attention_f16kv_64x1024x512", 2)]


def _representative_record(mod):
    """A record shaped like a full default run's (every field at its full length)."""
    kern = []
    for i, (name, cfg) in enumerate(KERNEL_LINES):
        shape = {"us_per_launch": 12.345, "bytes": 123456789, "GBps": 4567.8, "frac_of_peak": 0.5678,
                 "calls_per_config": 24, "rows": 65536, "rows_per_s": 123456789012.0}
        cpu = {"bytes": 123456789, "rows": 65536, "best_GBps": 2.345 + i,
               **{f"t{t}": {"us": 1234.56, "GBps": 1.234, "rows_per_s": 1234567.0, "cv": 0.0123,
                            "calls_per_rep": 3} for t in (1, 16)}}
        kern.append({"kernel": name, "config": cfg, "stated_shape": shape,
                     "replicated": dict(shape, instances=512, us=1234.56), "cpu": cpu,
                     "vs_cpu_best": 1234.5})
    full = [{"kv_len": kv, "us_per_step": 1106.9, "tokens_per_s": 57819.0, "frac_of_peak": 0.3871,
             "launches": 292, "bytes_per_step": 3430000000} for kv in (1024, 2048)]
    conv = {"roofline": {"frac": 0.0948, "achieved": 236.9, "peak": 2500.0, "flops": 914227200000.0},
            "generator": {"decoder": {"us": 3761.2, "eager_us": 3700.5, "launches": 103}},
            "stages": [{}] * 5}
    return {
        "metric": mod.METRIC, "value": 1389.51, "unit": "GB/s", "n_gpus": 1, "steps": 200,
        "warmup": 20, "ms_per_step": 0.01639, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded normal activations / parameters, uniform ids and positions)",
        "config": {"workload": "t2s_decode_step_epilogues", "batch": 64, "d_model": 512,
                   "ffn": 2048, "layers": 24, "storage": "f16", "launches_per_step": 1,
                   "fused": True, "bytes_per_step": 22774784, "us_per_step": 16.391,
                   "frac_of_peak": 0.17368, "rows_per_s": 285198000.0, "tokens_per_s": 3904582.0,
                   "graph": False, "one_node_graph_us_per_step": 34.141,
                   "per_op_graph_us_per_step": 144.041, "per_op_graph_launches": 73},
        "roofline": {"kernel": "t2s_step_fused [B=64, D=512, FF=2048, 24 layers] f16",
                     "bound": "hbm", "achieved": 1580.3, "peak": 8000.0, "unit": "GB/s",
                     "frac": 0.19754, "traffic": 23456789, "bytes_per_launch": 22774784,
                     "us_per_launch": 14.412, "rows_per_s": 324340000.0,
                     "traffic_detail": {"bytes": 23456789, "fetch_kib": 12345.678,
                                        "write_kib": 12345.678, "fetch_scale": 1.0123,
                                        "write_scale": 0.9876}},
        "cpu_baseline": {"value": 1.234, "unit": "GB/s", "cores": 16, "kind": "port",
                         "sample": "median of 9 repetitions x 12 decode steps (B=64, 24 layers, fp16 "
                                   "storage) of the oracle's C restatement, rows split over 16 "
                                   "threads; 2 warm-up steps",
                         "us_per_step": 12345.6, "cv": 0.0123, "rows_per_s": 1234567.0,
                         "single_thread_us_per_step": 123456.7, "single_thread_cv": 0.0123,
                         "cpu_model": "AMD EPYC 9575F 64-Core Processor",
                         "logical_cpus_allowed": 16, "hardware_threads": 256,
                         "physical_cores_on_host": 128, "threads_used": 16},
        "per_op": {"residual_layernorm": {"us_per_launch": 1.9}}, "copy_GBps": 5000.0,
        "kernels": kern, "t2s_whole_decode_step": full, "sovits_conv": conv,
        "detail_file": "gpurun_out/bench_detail.json",
    }


def test_headline_line_fits_the_captured_tail_and_keeps_its_keys():
    """The driver keeps only the end of the output: the last line must stay short and carry the
    metric, the roofline of the dominant kernel and the CPU baseline."""
    import json
    mod = _bench()
    rec = _representative_record(mod)
    s = mod.headline_line(rec)
    assert "\n" not in s
    assert len(s) <= mod.HEADLINE_MAX_CHARS <= 3000
    line = json.loads(s)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "dtype",
                "config", "roofline", "cpu_baseline", "higher_is_better", "vs_baseline"):
        assert key in line, key
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in line["roofline"], key
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in line["cpu_baseline"], key
    # a full record still fits with every summary
    assert set(line["configs"]) == {"1", "2", "3", "4", "5"}
    assert line["configs"]["2"]["lines"] == sum(c == 2 for _, c in KERNEL_LINES)
    assert line["configs"]["4"]["cpu_best_GBps"] is not None
    assert set(line["whole_decode_step"]) == {"kv1024", "kv2048"}
    assert line["sovits"]["decoder_graph_us"] == 3761.2
    assert line["sovits"]["decoder_eager_us"] == 3700.5
    assert line["sovits"]["decoder_frac_mfma"] == round(914227200000.0 / 3761.2 / 1e6 / 2500.0, 4)
    # the suite itself stays out of the line
    for key in ("kernels", "sovits_conv", "t2s_whole_decode_step", "per_op"):
        assert key not in line


def test_headline_line_drops_summaries_before_exceeding_the_bound():
    import json
    mod = _bench()
    rec = _representative_record(mod)
    rec["data"] = "x" * 2000  # a record whose headline keys alone take most of the bound
    s = mod.headline_line(rec)
    line = json.loads(s)
    assert "roofline" in line and "cpu_baseline" in line
    assert "configs" not in line or len(s) <= mod.HEADLINE_MAX_CHARS


def test_detail_file_holds_the_full_record(tmp_path):
    import json
    mod = _bench()
    rec = _representative_record(mod)
    path = tmp_path / "sub" / "detail.json"
    assert mod.write_detail(rec, str(path))
    back = json.loads(path.read_text())
    assert len(back["kernels"]) == len(KERNEL_LINES)
    assert back["roofline"]["frac"] == rec["roofline"]["frac"]
    assert mod.write_detail(rec, "") is None


def test_cpu_band_split_covers_every_item_once():
    mod = _bench()
    for n in (1, 5, 64, 499, 31999, 7680000):
        for parts in (1, 3, 16, 64):
            bands = mod._bands(n, parts)
            assert len(bands) <= parts
            assert bands[0][0] == 0 and bands[-1][1] == n
            assert all(lo < hi for lo, hi in bands)
            assert all(a[1] == b[0] for a, b in zip(bands, bands[1:]))
