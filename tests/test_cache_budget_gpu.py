"""The HBM weight cache over its budget (ggml-rocket.cpp:4297-4528: a weight that does not fit
the cache budget streams per call): with CACHE_MB=1 no weight fits, so every MUL_MAT decodes its
weight into per-call scratch on route "mt" (QUANT_RESIDENT=1 included) and still matches the
oracle; a named expert stack past the budget is streamed, and moe_stats counts each routed
expert once over the backend's life (ggml-rocket.h:39-57); the teardown report names the outcome.
Knobs are read once per process, so this runs in a child process."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_weight_cache_over_budget_streams(torch_cuda):
    env = {k: v for k, v in os.environ.items() if not k.startswith(("MI355X_", "ROCKET_"))}
    env.update({"MI355X_CACHE_MB": "1", "MI355X_MOE": "1"})
    r = subprocess.run([sys.executable, os.path.join(HERE, "cache_budget_child.py")], capture_output=True,
                       text=True, env=env, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0
    out = json.loads(r.stdout.strip().splitlines()[-1])
    for k in ("q4k_0", "q4k_1", "f16_0", "f16_1"):
        assert out[k]["status"] == 0 and out[k]["nbad"] == 0 and out[k]["range_err"] <= 1e-2, k
    assert out["routes"] == {"mt": 4, "prepacked": 0, "prepacked-q": 0}
    assert out["cpu_fallbacks"] == 0 and out["cpu_fallbacks_end"] == 0
    for rep in range(3):
        m = out[f"moe_{rep}"]
        assert m["status"] == 0 and m["nbad"] == 0 and m["range_err"] <= 1e-2
        assert m["stats"] == [0, m["distinct"]], m   # streamed experts, distinct over the life
    # the same ids again count nothing new; new ids add only the experts not seen before
    assert out["moe_1"]["stats"] == out["moe_0"]["stats"]
    assert out["moe_2"]["distinct"] > out["moe_0"]["distinct"]
    # the teardown report says the cache held nothing and why (ggml-rocket.cpp:5185-5303)
    report = [ln for ln in r.stderr.splitlines() if "[mi355x]" in ln]
    assert any("[f16-resident] 0 weights resident" in ln and "0% resident" in ln for ln in report), report
    assert any("[f16-resident] first weight turned away at 0.0 MB cached" in ln and "1 MB budget" in ln
               for ln in report), report
    assert any("[moe] 0 weights resident" in ln and "1 run from per-call uploads" in ln for ln in report), report
