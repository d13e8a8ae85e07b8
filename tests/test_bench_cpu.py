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
