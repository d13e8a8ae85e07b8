"""bench.py's contract on the host: more than one GPU is refused with a message, and the
CPU-baseline helpers time the oracle on bounded samples (no device work)."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_exits_with_a_message():
    out = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 2
    line = json.loads(out.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_cpu_baselines_attach_to_every_gemm_and_permutation_workload():
    sys.path.insert(0, str(REPO))
    import bench
    g = np.random.default_rng(3)

    def gm(m, n, k, a_t=False, b_t=False, batch=1, beta=0.0):
        a = g.uniform(-1, 1, batch * m * k).astype(np.float32)
        b = g.uniform(-1, 1, batch * k * n).astype(np.float32)
        return {"_host": (a, b), "_geom": (m, n, k, a_t, b_t, batch, beta)}

    res = {"c1": gm(24, 16, 8), "c3": gm(8, 8, 8, b_t=True, batch=3),
           "c5": {"parts": [gm(8, 12, 4), gm(8, 4, 12, b_t=True), gm(4, 12, 8, a_t=True, beta=1.0)]},
           "c2b": {"_host": g.uniform(-1, 1, 60).astype(np.float32), "_geom": ([3, 4, 5], [2, 0, 1])},
           "copy": {"gbs": 1.0}}
    bench.attach_cpu_baselines(res, 2)
    for name in ("c1", "c3", "c5", "c2b"):
        for key in ("cpu_baseline", "cpu_baseline_parallel"):
            cb = res[name][key]
            assert cb["value"] > 0 and cb["kind"] == "port" and cb["sample"], (name, key)
        assert "_host" not in res[name]
    assert res["c5"]["parts"][2]["cpu_baseline"]["unit"] == "TFLOP/s"
    assert res["c2b"]["cpu_baseline_parallel"]["cores"] == 2
    assert "cpu_baseline" not in res["copy"]


def _stub_results():
    """A result set shaped like a full run's: every workload, long kernel lists and samples."""
    cpu = {"value": 0.000207, "unit": "TFLOP/s", "cores": 1, "kind": "port",
           "sample": "48 of 4096 output rows, literal k-order loop (3 runs, 0.81 s)"}
    cpu_par = dict(cpu, cores=16, sample="4096 of 4096 output rows, bit-identical "
                                         "loop-interchanged variant on 16 threads (1.20 s)")
    plan = {"kind": "tiled", "kernel": "pipelined", "tile": [256, 128], "a_mode": "k",
            "b_mode": "mn", "splits": 1, "workgroups": 512}

    def gemm(tf):
        return {"name": "gemm x" * 8, "ms": 0.9661, "ms_median": 0.9662, "ms_best": 0.9601,
                "host_ms": 0.01, "tflops": tf, "frac": tf / 157.3, "plan": plan,
                "kernels": ["gemm_f32_pl<0, 1, 16, 4, 1>", "reduce_f32"],
                "cpu_baseline": cpu, "cpu_baseline_parallel": cpu_par}

    def perm(gbs):
        return {"name": "perm", "ms": 0.1745, "gbs": gbs, "frac": gbs / 8000.0,
                "plan": {"kind": "tile", "vector": True, "workgroups": 8192,
                         "shape": [256, 524288]}, "kernels": ["perm_tile_w1_v128_stream"],
                "cpu_baseline": dict(cpu, unit="GB/s"), "cpu_baseline_parallel": cpu_par}

    def other(bound):
        roof = ({"bound": "mfma", "achieved": 114.2, "peak": 157.3, "unit": "TFLOP/s",
                 "frac": 0.726} if bound == "mfma" else
                {"bound": "hbm", "achieved": 4342.3, "peak": 8000.0, "unit": "GB/s",
                 "frac": 0.543})
        return {"name": "other", "ms": 0.2142, "tflops": 114.2, "gbs": 297.4, "roofline": roof,
                "plan": plan, "kernels": ["gemm_f32_pl_n64<K,MN>"], "cpu_baseline": cpu}

    res = {k: gemm(140.0) for k in ("gemm4096", "sq1024", "sq2048", "c1", "c3", "c4")}
    res["c5"] = {"name": "C5", "ms": 12.0, "tflops": 137.0, "frac": 0.87,
                 "parts": [gemm(137.0)] * 3, "cpu_baseline": cpu, "cpu_baseline_parallel": cpu_par}
    for k in ("c2a", "c2b", "c2b_1g"):
        res[k] = perm(6100.0)
    res["copy"] = {"name": "copy", "gbs": 6683.7}
    res["t8191"] = dict(perm(5325.0), copy_gbs=6718.0, ratio_vs_copy=0.79)
    res["floor"] = {"name": "floor", "ms": 0.0099, "ms_graph": 0.0032, "kernels": ["zero_f32"]}
    res["f16"] = {"name": "f16", "ms": 2.24, "tflops": 61.3, "frac_f64_mfma": 0.78,
                  "cpu_baseline": cpu}
    res["o_f16_2048"] = dict(res["f16"])
    for k in ("o_t2048", "o_rank4"):
        res[k] = other("mfma")
    for k in ("o_batched", "o_dot", "o_32k1m", "o_rank1"):
        res[k] = other("hbm")
    train = {op: {"ms": 0.2, "gbs": 5900.0, "frac": 0.74, "bytes": 1 << 29, "kernel": op,
                  "cpu_baseline": dict(cpu, unit="GB/s")}
             for op in ("gelu", "gelu_backward", "add_bias", "bias_grad", "mse_grad", "sgd_step",
                        "convert_f32_bf16", "convert_bf16_f32")}
    bgemm16 = {"name": "bgemm16", "ms": 3.3, "tterms": 20.7, "tflops_vector": 41.4,
               "frac_vector": 0.263, "kernel": "gemm16_seq<0, 8>", "cpu_baseline": cpu}
    return res, train, bgemm16


def test_headline_line_is_compact_and_carries_the_required_keys():
    sys.path.insert(0, str(REPO))
    import bench

    class Args:
        steps, warmup, warmup_ms, no_cpu = 20, 50, 30.0, False
    res, train, bgemm16 = _stub_results()
    line = bench.headline_line(res, Args, train, bgemm16, "gpurun_out/bench_detail.json")
    text = json.dumps(line)
    assert len(text) <= bench.LINE_LIMIT < 4096
    parsed = json.loads(text)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "dtype",
                "data", "config", "roofline", "cpu_baseline", "cpu_baseline_parallel", "permute",
                "configs_summary", "higher_is_better", "scaling", "vs_baseline"):
        assert key in parsed, key
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in parsed["roofline"], key
    assert parsed["roofline"]["frac"] == round(140.0 / 157.3, 4)
    assert parsed["value"] == 140.0 and parsed["ms_per_step"] == 0.9661
    summ = parsed["configs_summary"]
    for name in ("c1", "c2a", "c2b", "c2b_1g", "c3", "c4", "c5", "o_rank4", "bgemm16"):
        assert len(summ[name]) == 3, name
    assert summ["c2b_1g"] == [6100.0, "GB/s", round(6100.0 / 8000.0, 4)]
    assert summ["bgemm16"][2] <= 1.0  # priced against the published fp32 vector peak
    # The detail record keeps what the line leaves out.
    detail = bench.detail_record(res, Args, train, bgemm16)
    assert detail["configs"]["c5"]["parts"][0]["plan"]["workgroups"] == 512


def test_headline_line_sheds_optional_parts_before_exceeding_the_limit():
    sys.path.insert(0, str(REPO))
    import bench

    class Args:
        steps, warmup, warmup_ms, no_cpu = 20, 50, 30.0, False
    res, train, bgemm16 = _stub_results()
    for i in range(200):  # far more workloads than any run has
        res[f"x{i}"] = res["c1"]
    old = bench.SUMMARY_ORDER
    try:
        bench.SUMMARY_ORDER = tuple(res)
        line = bench.headline_line(res, Args, train, bgemm16, "d.json")
    finally:
        bench.SUMMARY_ORDER = old
    assert len(json.dumps(line)) <= bench.LINE_LIMIT
    assert line["value"] == 140.0 and "roofline" in line and "cpu_baseline" in line
