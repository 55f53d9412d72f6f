"""Child process of test_cache_budget_gpu.py: knobs are read once per process, so the
over-budget weight cache runs here with MI355X_CACHE_MB=1 set by the parent. Prints one JSON
line with what the parent asserts."""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(HERE), os.path.join(os.path.dirname(HERE), "ggml-rocket_amd"), HERE]

import numpy as np  # noqa: E402

import ggml_mi355x as mx  # noqa: E402
from oracle import oracle as O  # noqa: E402
from bars import compare  # noqa: E402


def mul_mat(be, wt, payload, K, N, M, name, seed):
    g = mx.Graph()
    W = g.new_tensor(wt, [K, N], name)
    X = g.new_tensor(mx.F32, [K, M])
    Xf = O.fill_normal((M, K), seed)
    g.set(W, payload), g.set(X, Xf)
    d = g.mul_mat(W, X)
    st = be.compute([d])
    got = g.get(d, np.float32, (M, N))
    ref = O.mul_mat(wt, payload, Xf, N, K)
    return st, compare(ref, got)


def main():
    out = {}
    be = mx.Backend()
    be.set_quant_resident(1)
    K, N, M = 2048, 1024, 512             # 4 MB of fp16: past the 1 MB budget
    Q = O.quantize(O.Q4_K, O.fill_normal((N, K), 880, 0.0, 0.02))
    F = O.f32_to_f16_bits(O.fill_normal((N, K), 881, 0.0, 0.02))
    for rep in range(2):                   # the second call finds nothing cached either
        st, r = mul_mat(be, O.Q4_K, Q, K, N, M, "blk.0.ffn_up.weight", 882 + rep)
        out[f"q4k_{rep}"] = {"status": st, "nbad": r["nbad"], "range_err": r["range_err"]}
        st, r = mul_mat(be, O.F16, F, K, N, M, "blk.0.ffn_gate.weight", 884 + rep)
        out[f"f16_{rep}"] = {"status": st, "nbad": r["nbad"], "range_err": r["range_err"]}
    out["routes"] = {k: be.route_ops(k) for k in ("mt", "prepacked", "prepacked-q")}
    out["cpu_fallbacks"] = be.cpu_fallbacks()

    # a named expert stack past the budget: streamed, each routed expert counted once
    E, U, T, Ke, Ne = 16, 2, 64, 512, 256
    P = O.quantize(O.Q4_K, O.fill_normal((E, Ne, Ke), 886, 0.0, 0.02))
    seen = set()
    for rep, (lo, hi) in enumerate(((0, 6), (0, 6), (4, 10))):
        g = mx.Graph()
        a = g.new_tensor(mx.Q4_K, [Ke, Ne, E], "blk.0.ffn_down_exps.weight")
        b = g.new_tensor(mx.F32, [Ke, 1, T])
        ids = g.new_tensor(mx.I32, [U, T])
        Xm = O.fill_normal((T, 1, Ke), 887 + rep)
        iv = (lo + (np.arange(T)[:, None] * 3 + np.arange(U)[None, :]) % (hi - lo)).astype(np.int32)
        g.set(a, P), g.set(b, Xm), g.set(ids, iv)
        d = g.mul_mat_id(a, b, ids)
        st = be.compute([d])
        r = compare(O.mul_mat_id(O.Q4_K, P, Ke, Ne, E, Xm, 1, iv), g.get(d, np.float32, (T, U, Ne)))
        seen |= set(iv.ravel().tolist())
        out[f"moe_{rep}"] = {"status": st, "nbad": r["nbad"], "range_err": r["range_err"],
                             "stats": list(be.moe_stats()), "distinct": len(seen)}
    out["cpu_fallbacks_end"] = be.cpu_fallbacks()
    be.free()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
