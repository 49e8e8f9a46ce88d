"""bench.py's output contract, on the CPU: the stdout line the driver parses (size and required keys), the CSV's
columns (apps/bench/bench.cpp:112-113's, in order, then the GPU columns), and that every bench.py command the
profiles under profiles/ were taken with is one the current argument parser accepts."""
import csv
import glob
import importlib.util
import json
import os
import re
import shlex

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


# every row key bench.py's default run produces (build_rows, then build_rows(split=True))
ROW_KEYS = ["matmul512_nn", "matmul512_tn", "matmul512_nt", "mlp_forward", "mlp_backward", "conv1_forward",
            "conv1_forward_no_alive", "conv1_backward", "pool1_forward", "conv1_pool1_forward", "pool1_backward",
            "conv1_forward_packed", "conv1_pool1_forward_packed", "conv1_backward_packed", "pool1_backward_packed",
            "conv2_forward", "conv2_backward", "attention_forward", "attention_backward", "attention_forward_causal",
            "attention_backward_causal", "matmul_1024x1024x1024", "matmul_2048x2048x2048", "matmul_4096x4096x4096",
            "matmul_8192x8192x8192", "matmul_64x4096x4096", "matmul_4096x4096x64"]
SPLIT_KEYS = ["matmul512_nn_split", "matmul512_tn_split", "matmul512_nt_split", "mlp_forward_split",
              "mlp_backward_split", "matmul_64x4096x4096_split"]


def full_row(key, i):
    """A row as row_json writes it, with long fractional values and every optional field present."""
    row = {"cfg": 5, "key": key, "workload": "nn::matmul 8192x8192x8192 C = A B with a long description " * 2,
           "ms": 1.123456789 + i, "spread": 0.012345, "runs": 7, "tflops": 122.191234,
           "roofline": {"bound": "mfma", "achieved": 122.1915123, "peak": 157.3, "unit": "TFLOP/s",
                        "frac": 0.776812345},
           "bitwise_repeat": True, "bitwise_vs_nn_cpp": i % 2 == 0, "maxabs_vs_nn_cpp": 1.2345e-7,
           "cpu_baseline": {"ms": 606.0233123, "threads": 16, "runs": 3, "spread": 0.0069, "speedup_gpu": 67.3},
           "cpu_1thread": {"ms": 8020.4746123, "threads": 1, "runs": 1, "spread": 0.0, "speedup_gpu": 891.3}}
    if key.endswith("_causal"):
        row["roofline"]["useful_frac"] = 0.4012345
    if key.endswith("_packed"):
        row["bitwise_vs_byte_form"] = True
    return row


def full_result():
    return {
        "metric": "fp32 GEMM TFLOP/s @4096^3 + % MI355X fp32 MFMA peak; fused-op GB/s",
        "value": 123.456, "unit": "TFLOP/s", "n_gpus": 1, "steps": 20, "warmup": 5, "settle_launches": 412,
        "ms_per_step": 1.12345, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: the reference's seeded streams (std::mt19937(seed) + uniform_real_distribution<float>; "
                "N(0,1) from numpy's PCG64 where BASELINE.json asks for normal values); both sides get the same buffers",
        "config": {"workload": "sgemm 4096x4096x4096 NN fp32 (BASELINE config 5)", "m": 4096, "n": 4096, "k": 4096,
                   "trans_a": False, "trans_b": False, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": 124.9, "peak": 157.3, "unit": "TFLOP/s", "frac": 0.794,
                     "traffic": 604138031.0},
        "cpu_baseline": {"value": 1.842, "unit": "TFLOP/s", "cores": 16, "kind": "reference",
                         "sample": "nn::matmul 4096^3, nn-cpp NN_NATIVE AVX2 build (oracle/_ref), same seed-4 "
                                   "inputs, 16 threads pinned 1/physical core of AMD EPYC 9575F 64-Core Processor "
                                   "(performance), median of 15 after 1 warm-up"},
        "cpu_setup": {"cpu": "AMD EPYC", "pinned_to": list(range(64))},
        "fused_op": {"workload": "conv1", "value": 2165.4, "unit": "GB/s", "us_per_launch": 6.118,
                     "algorithmic_bytes": 13247744, "roofline": {"bound": "hbm", "peak": 8000.0, "unit": "GB/s",
                                                                 "frac": 0.2707},
                     "fill_floor": {"us_per_launch": 3.812, "conv1_frac_of_floor": 0.6412}},
        "configs": [full_row(k, i) for i, k in enumerate(ROW_KEYS)],
        "configs_split_depth": [full_row(k, i) for i, k in enumerate(SPLIT_KEYS)],
        "next_rows": [full_row("layernorm_attention_acts_backward", i) for i in range(6)],
        "workloads": [{"workload": w, "batch": 256,
                       "gpu": {"forward_ms": 0.1, "backward_ms": 0.2, "total_ms": 0.312345, "spread": 0.01,
                               "runs": 15},
                       "cpu": {"forward_ms": 1.1, "backward_ms": 1.7, "total_ms": 2.80512, "spread": 0.02,
                               "runs": 15, "threads": 16},
                       "bitwise_vs_nn_cpp": True, "speedup_gpu": 4.2}
                      for w in ("mlp_wide", "cnn_mnist", "transformer_tiny")],
        "full_rows": "gpurun_out/bench_full.json",
    }


def test_stdout_line_fits_and_carries_the_contract(bench):
    text = bench.compact_line(full_result())
    assert "\n" not in text
    assert len(text.encode()) <= bench.LINE_LIMIT
    line = json.loads(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["roofline"]["traffic"] == 604138031.0
    assert set(line["roofline"]) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}
    assert set(line["cpu_baseline"]) >= {"value", "unit", "cores", "kind", "sample"}
    # the packed-flag rows travel as their time and check in fused_op
    assert list(line["configs"]) == [k for k in ROW_KEYS if not k.endswith("_packed")]
    assert list(line["fused_op"]["packed_us"]) == ["fwd", "fwd_pool", "bwd", "pool_bwd", "bitwise"]
    assert line["fused_op"]["packed_us"]["bitwise"] is True
    assert list(line["configs_split_depth"]) == SPLIT_KEYS
    for r in line["configs"].values():
        assert set(r) >= {"ms", "frac", "cpu_ms", "bitwise"}
    for r in line["configs_split_depth"].values():
        assert set(r) >= {"ms", "frac", "bitwise"}
    assert line["configs"]["attention_backward_causal"]["useful_frac"] == 0.4012
    # an exact row is bitwise only when it repeats and equals nn-cpp; a split row only has to repeat
    assert line["configs"]["matmul512_nn"]["bitwise"] is True and line["configs"]["matmul512_tn"]["bitwise"] is False
    assert all(r["bitwise"] for r in line["configs_split_depth"].values())
    assert len(text.encode()) <= bench.LINE_LIMIT - 200  # room for longer CPU model names and more digits
    assert line["workloads"][0]["gpu_ms"] == 0.3123 and "optimizer" in line["workloads_note"]
    assert line["fused_op"]["frac_of_fill_floor"] == 0.6412


def test_stdout_line_refuses_to_outgrow_the_limit(bench):
    big = full_result()
    big["configs"] = [full_row(f"{k}_{j}", i) for j in range(4) for i, k in enumerate(ROW_KEYS)]
    with pytest.raises(ValueError):
        bench.compact_line(big)
    # outside the test the line sheds its optional parts instead of failing the run
    text = bench.compact_line(dict(big, configs=big["configs"][:30]), strict=False)
    line = json.loads(text)
    assert len(text.encode()) <= bench.LINE_LIMIT and "value" in line and "roofline" in line


class _Row:
    def __init__(self, key, cfg, flops, bound, result):
        self.key, self.cfg, self.flops, self.bound, self.result = key, cfg, flops, bound, result


def test_csv_has_the_reference_columns_in_order(bench, tmp_path):
    res = full_row("matmul512_nn", 0)
    res["roofline"]["bound"] = "mfma"
    rows = [_Row("matmul512_nn", 1, 2.0 * 512 ** 3, "mfma", res),
            _Row("conv1_backward", 3, 1.0e8, "hbm", dict(full_row("conv1_backward", 1), gbps=500.0))]
    path = tmp_path / "rows.csv"
    wl = full_result()["workloads"]
    bench.write_csv(str(path), rows, None, wl)
    with open(path) as fh:
        table = list(csv.reader(fh))
    reference_cols = ["config", "label", "threads", "benchmark", "size", "forward_ms", "backward_ms", "optim_ms",
                      "total_ms", "gflops", "spread", "runs"]  # apps/bench/bench.cpp:112-113
    assert table[0][:12] == reference_cols
    assert table[0][12:] == ["tflops", "gbps", "roofline_bound", "roofline_frac", "maxabs_err", "bitwise_repeat"]
    body = [dict(zip(table[0], r)) for r in table[1:]]
    # per row: the GPU line, the pinned CPU line, the 1-thread CPU line; then GPU and CPU lines per workload
    assert len(body) == 3 * 2 + 2 * len(wl)
    gpu = body[0]
    assert gpu["label"] == "gpu-mi355x" and gpu["benchmark"] == "matmul512_nn" and gpu["size"] == "512"
    assert float(gpu["forward_ms"]) == pytest.approx(res["ms"], rel=1e-5) and gpu["backward_ms"] == ""
    assert float(gpu["gflops"]) == pytest.approx(2.0 * 512 ** 3 / (res["ms"] * 1e6), rel=1e-5)
    assert body[1]["label"] == "native-pinned" and body[1]["threads"] == "16"
    assert body[2]["label"] == "native-1thread" and body[2]["threads"] == "1"
    back = body[3]
    assert back["size"] == "3" and bench.csv_size("matmul_64x4096x4096", 5) == "64x4096x4096"
    assert back["benchmark"] == "conv1_backward" and back["forward_ms"] == "" and back["backward_ms"] != ""
    assert body[6]["benchmark"] == "mlp_wide" and body[6]["optim_ms"] == ""


def _bench_commands():
    """Every `bench.py ...` invocation written in profiles/*.md, with its shell-level tail (redirections,
    comments) cut off and placeholders such as ROW given a real row key."""
    cmds = []
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        for line in open(path):
            m = re.search(r"bench\.py((?:\s+[^\s`|>#;)]+)*)", line)
            if not m or "python" not in line:
                continue
            argv = shlex.split(m.group(1))
            argv = ["conv1_backward" if a in ("ROW", "KEY") else a for a in argv]
            cmds.append((os.path.basename(path), argv))
    return cmds


def test_profiles_commands_parse(bench):
    cmds = _bench_commands()
    assert len(cmds) >= 10
    parser = bench.make_parser()
    for name, argv in cmds:
        try:
            parser.parse_args(argv)
        except SystemExit:
            pytest.fail(f"{name}: bench.py {' '.join(argv)} is rejected by the current bench.py")
