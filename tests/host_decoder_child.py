"""Child process of test_host_decoder_gpu.py: a decoder registered for a type the kernels do not
decode is process-wide, and MoE knobs are read once per process, so this runs on its own with
MI355X_MOE=1 set by the parent. Prints one JSON line with what the parent asserts.

The type is Q4_1 (ggml's { fp16 d; fp16 m; u8 qs[16]; } per 32 values, y = d * q + m; qs[j] low
nibble = value j, high nibble = value j + 16). The registered decoder stands in for ggml's
to_float, which the plugin registers in production; the expected results decode the same bytes
with the same formula in numpy, round the weight to fp16 as the device path does (the
reference's to_float then fp32_to_fp16_row, ggml-rocket.cpp:3894-3909) and take the fp64 GEMM."""
import ctypes
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(HERE), os.path.join(os.path.dirname(HERE), "ggml-rocket_amd"), HERE]

import numpy as np  # noqa: E402

import ggml_mi355x as mx  # noqa: E402
from oracle import oracle as O  # noqa: E402
from bars import compare  # noqa: E402


def q4_1_quantize(W):
    """[rows, K] f32 -> Q4_1 bytes [rows, K/32 * 20]."""
    rows, K = W.shape
    b = W.reshape(rows, K // 32, 32)
    lo, hi = b.min(axis=2), b.max(axis=2)
    d16 = ((hi - lo) / 15.0).astype(np.float16)
    m16 = lo.astype(np.float16)
    d = d16.astype(np.float32)
    q = np.clip(np.rint((b - m16.astype(np.float32)[..., None]) / np.where(d == 0, 1, d)[..., None]), 0, 15)
    q = q.astype(np.uint8)
    out = np.empty((rows, K // 32, 20), np.uint8)
    out[..., 0:2] = d16.view(np.uint8).reshape(rows, K // 32, 2)
    out[..., 2:4] = m16.view(np.uint8).reshape(rows, K // 32, 2)
    out[..., 4:20] = q[..., :16] | (q[..., 16:] << 4)
    return out.reshape(rows, -1)


def q4_1_decode(raw, n):
    blk = np.frombuffer(raw, np.uint8).reshape(n // 32, 20)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
    m = blk[:, 2:4].copy().view(np.float16).astype(np.float32)
    qs = blk[:, 4:20]
    q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float32)
    return (q * d + m).reshape(-1)


calls = [0]


def decoder(src, dst, n):
    calls[0] += 1
    y = q4_1_decode(ctypes.string_at(src, n // 32 * 20), n)
    np.ctypeslib.as_array(dst, shape=(n,))[:] = y


def main():
    out = {"register": mx.set_to_float(mx.Q4_1, 32, 20, decoder)}
    be = mx.Backend()
    K, N, M = 1024, 512, 512
    W = O.fill_normal((N, K), 890, 0.0, 0.02)
    P = q4_1_quantize(W)
    w16 = O.f32_to_f16_bits(q4_1_decode(P.tobytes(), N * K).reshape(N, K))
    for rep in range(2):                      # the second call finds the fp16 image cached
        g = mx.Graph()
        Wt = g.new_tensor(mx.Q4_1, [K, N], "blk.0.attn_output.weight")
        X = g.new_tensor(mx.F32, [K, M])
        Xf = O.fill_normal((M, K), 891 + rep)
        g.set(Wt, P), g.set(X, Xf)
        d = g.mul_mat(Wt, X)
        n0 = calls[0]
        st = be.compute([d])
        r = compare(O.mul_mat(O.F16, w16, Xf, N, K), g.get(d, np.float32, (M, N)))
        out[f"mm_{rep}"] = {"status": st, "nbad": r["nbad"], "range_err": r["range_err"],
                            "decoder_calls": calls[0] - n0}
    out["routes_mm"] = {k: be.route_ops(k) for k in ("prepacked-q", "mt", "prepacked")}

    # an expert stack of the same type (FORCED MoE claim in this process)
    E, U, T, Ke, Ne = 8, 2, 64, 512, 256
    Ws = O.fill_normal((E * Ne, Ke), 892, 0.0, 0.02)
    Ps = q4_1_quantize(Ws)
    s16 = O.f32_to_f16_bits(q4_1_decode(Ps.tobytes(), E * Ne * Ke).reshape(E, Ne, Ke))
    g = mx.Graph()
    a = g.new_tensor(mx.Q4_1, [Ke, Ne, E], "blk.0.ffn_up_exps.weight")
    b = g.new_tensor(mx.F32, [Ke, 1, T])
    ids = g.new_tensor(mx.I32, [U, T])
    Xm = O.fill_normal((T, 1, Ke), 893)
    iv = ((np.arange(T)[:, None] * 3 + np.arange(U)[None, :]) % E).astype(np.int32)
    g.set(a, Ps), g.set(b, Xm), g.set(ids, iv)
    d = g.mul_mat_id(a, b, ids)
    st = be.compute([d])
    r = compare(O.mul_mat_id(O.F16, s16, Ke, Ne, E, Xm, 1, iv), g.get(d, np.float32, (T, U, Ne)))
    out["moe"] = {"status": st, "nbad": r["nbad"], "range_err": r["range_err"]}
    # the claim of such a stack at the claim floor of 512 tokens
    gc = mx.Graph(alloc=False)
    dc = gc.mul_mat_id(gc.new_tensor(mx.Q4_1, [Ke, Ne, E], "blk.0.ffn_gate_exps.weight"),
                       gc.new_tensor(mx.F32, [Ke, 1, 512]), gc.new_tensor(mx.I32, [U, 512]))
    out["moe_supported"] = mx.supports_op(dc)

    # the CPU fallback decodes through the same registered decoder (fp64 on the f32 values)
    be.inject_faults("gemm", 1)
    g = mx.Graph()
    Wt = g.new_tensor(mx.Q4_1, [K, N], "blk.1.attn_output.weight")
    X = g.new_tensor(mx.F32, [K, M])
    Xf = O.fill_normal((M, K), 894)
    g.set(Wt, P), g.set(X, Xf)
    d = g.mul_mat(Wt, X)
    st = be.compute([d])
    wf = q4_1_decode(P.tobytes(), N * K).reshape(N, K).astype(np.float32)
    r = compare(O.mul_mat(O.F32, wf, Xf, N, K), g.get(d, np.float32, (M, N)))
    out["fallback"] = {"status": st, "nbad": r["nbad"], "range_err": r["range_err"]}
    out["cpu_fallbacks"] = be.cpu_fallbacks()
    be.free()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
