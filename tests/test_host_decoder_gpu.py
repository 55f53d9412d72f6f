"""A quantized type the kernels do not decode, through a registered host decoder
(mi355x_backend_set_to_float; the plugin registers ggml's to_float for every quantized type, as
the reference decodes every quant type through it, ggml-rocket.cpp:3894-3909): MUL_MAT on the
fp16 image in the HBM cache (route "prepacked-q", decoded once, reused by the next call),
MUL_MAT_ID on an expert stack of the type, and the CPU fallback, each against the fp64 oracle on
the decoded weight. Runs in a child process (the registration is process-wide)."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_registered_host_decoder(torch_cuda):
    env = {k: v for k, v in os.environ.items() if not k.startswith(("MI355X_", "ROCKET_"))}
    env.update({"MI355X_MOE": "1"})
    r = subprocess.run([sys.executable, os.path.join(HERE, "host_decoder_child.py")], capture_output=True,
                       text=True, env=env, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["register"] == 0
    for k in ("mm_0", "mm_1", "moe", "fallback"):
        assert out[k]["status"] == 0 and out[k]["nbad"] == 0 and out[k]["range_err"] <= 1e-2, (k, out[k])
    assert out["mm_0"]["decoder_calls"] > 0 and out["mm_1"]["decoder_calls"] == 0, "decoded once, then cached"
    assert out["routes_mm"] == {"prepacked-q": 2, "mt": 0, "prepacked": 0}
    assert out["moe_supported"]
    assert out["cpu_fallbacks"] == 1
