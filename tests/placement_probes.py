"""Metadata-only placement probes (no data, no device), the helpers of test-rocket-placement.cpp
(34-145) on the backend's descriptor API. Also runnable as a child process:
`python placement_probes.py <mode>` prints a JSON list of [label, expected, got] rows, so that
knobs read once per process can be set per mode in a fresh environment (the reference forks a
child per knob configuration for the same reason, 374-385)."""
import ctypes
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.dirname(HERE), os.path.join(os.path.dirname(HERE), "ggml-rocket_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import ggml_mi355x as mx  # noqa: E402

PREC_F32, PREC_BF16, PREC_F16, PREC_Q8, PREC_Q4 = 10, 15, 20, 30, 40


def mm_supported(K, N, M, wt, slot=None, value=0):
    g = mx.Graph(alloc=False)
    W = g.new_tensor(wt, [K, N])
    X = g.new_tensor(mx.F32, [K, M])
    d = g.mul_mat(W, X)
    if slot is not None:
        d.op_params[slot] = value
    return mx.supports_op(d)


def mm_computed_w_supported(K, N, M):
    g = mx.Graph(alloc=False)
    W0 = g.new_tensor(mx.F16, [K, N])
    W = g.op(mx.F16, [K, N], mx.OP_SCALE, (W0,))   # src0 computed, not a leaf
    X = g.new_tensor(mx.F32, [K, M])
    return mx.supports_op(g.mul_mat(W, X))


def add_offloaded(K, M):
    g = mx.Graph(alloc=False)
    A = g.new_tensor(mx.F32, [K, M])
    B = g.new_tensor(mx.F32, [K, M])
    return mx.offload_op(g.op(mx.F32, [K, M], mx.OP_ADD, (A, B)))


def mm_offloaded(K, N, M):
    g = mx.Graph(alloc=False)
    return mx.offload_op(g.mul_mat(g.new_tensor(mx.F16, [K, N]), g.new_tensor(mx.F32, [K, M])))


def fa_supported(head_dim, n_tokens, n_head, n_kv, n_kv_heads, kv_t, max_bias, acc=0, dv=None):
    g = mx.Graph(alloc=False)
    q = g.new_tensor(mx.F32, [head_dim, n_tokens, n_head, 1])
    k = g.new_tensor(kv_t, [head_dim, n_kv, n_kv_heads, 1])
    v = g.new_tensor(kv_t, [dv or head_dim, n_kv, n_kv_heads, 1])
    pad = ((n_tokens + 31) // 32) * 32
    m = g.new_tensor(mx.F16, [n_kv, pad])
    d = g.flash_attn_ext(q, k, v, m, 1.0, max_bias, 0.0, acc)
    return mx.supports_op(d)


def moe_supported(K, N, n_expert, n_tokens, wt, name, n_used=4, src1_prec=0, buffer=None):
    g = mx.Graph(alloc=False)
    a = g.new_tensor(wt, [K, N, n_expert], name)
    if buffer is not None:
        a.buffer_kind = mx.BUF_HOST
        a.buffer_id, a.buffer_size = buffer
    b = g.new_tensor(mx.F32, [K, 1, n_tokens])
    ids = g.new_tensor(mx.I32, [n_used, n_tokens])
    d = g.mul_mat_id(a, b, ids)
    if src1_prec:
        d.op_params[3] = src1_prec
    return mx.supports_op(d)


EK, EN, NE, NT = 2880, 2880, 8, 512      # gpt-oss-20b expert GEMM
DK, DN = 2048, 1408                      # DeepSeek-V2-Lite expert GEMM


def moe_auto_rows():
    r = []
    r.append(("MoE: Q8_0 experts, src1 F32 declared -> CPU", False,
              moe_supported(EK, EN, NE, NT, mx.Q8_0, "blk.20.ffn_down_exps.weight", 4, PREC_F32)))
    # MI355X: the expert route keeps activations in fp16 (no int8 requant), so an F16
    # declaration is met; the reference's int8 route declines it (ggml-rocket.cpp:7360-7363).
    r.append(("MoE: Q8_0 experts, src1 F16 declared -> offload (fp16 activations here)", True,
              moe_supported(EK, EN, NE, NT, mx.Q8_0, "blk.21.ffn_down_exps.weight", 4, PREC_F16)))
    r.append(("MoE: Q8_0 experts, fits budget -> offload", True,
              moe_supported(EK, EN, NE, NT, mx.Q8_0, "blk.0.ffn_gate_exps.weight")))
    r.append(("MoE: F16 experts -> CPU (no dequant to delete)", False,
              moe_supported(EK, EN, NE, NT, mx.F16, "blk.1.ffn_gate_exps.weight")))
    r.append(("MoE: unnamed expert stack -> CPU", False, moe_supported(EK, EN, NE, NT, mx.Q8_0, None)))
    r.append(("MoE: n_tokens=1 (decode) -> CPU", False,
              moe_supported(EK, EN, NE, 1, mx.Q8_0, "blk.2.ffn_gate_exps.weight")))
    r.append(("MoE: K%32!=0 (K=80) -> CPU", False, moe_supported(80, EN, NE, NT, mx.Q8_0, "blk.3.ffn_gate_exps.weight")))
    r.append(("MoE: 4-of-32, M_e=64 (at granule) -> offload", True,
              moe_supported(EK, EN, 32, 512, mx.Q8_0, "blk.4.ffn_gate_exps.weight", 4)))
    r.append(("MoE: 6-of-64, M_e=48 (under granule) -> CPU", False,
              moe_supported(DK, DN, 64, 512, mx.Q8_0, "blk.5.ffn_gate_exps.weight", 6)))
    r.append(("MoE: 6-of-64, M_e=192 at pp2048 -> offload", True,
              moe_supported(DK, DN, 64, 2048, mx.Q8_0, "blk.6.ffn_gate_exps.weight", 6)))
    r.append(("MoE: 4-of-32 M_e=96, 796 MMAC/dispatch -> offload", True,
              moe_supported(EK, EN, 32, 768, mx.Q8_0, "blk.7.ffn_gate_exps.weight", 4)))
    r.append(("MoE: 6-of-64 M_e=72, 208 MMAC/dispatch -> CPU (under the work floor)", False,
              moe_supported(DK, DN, 64, 768, mx.Q8_0, "blk.10.ffn_gate_exps.weight", 6)))
    r.append(("MoE: 6-of-64 M_e=96, 277 MMAC/dispatch -> CPU (the boundary cell)", False,
              moe_supported(DK, DN, 64, 1024, mx.Q8_0, "blk.8.ffn_gate_exps.weight", 6)))
    r.append(("MoE: 6-of-64 M_e=144, 415 MMAC/dispatch -> offload", True,
              moe_supported(DK, DN, 64, 1536, mx.Q8_0, "blk.9.ffn_gate_exps.weight", 6)))
    return r


def moe_budget_rows():
    return [("MoE: stack over the budget (1 MB) -> CPU", False,
             moe_supported(EK, EN, 8, 512, mx.Q8_0, "blk.0.ffn_gate_exps.weight"))]


def moe_off_rows():
    return [("MoE: Q8_0 experts, MOE=0 -> CPU", False,
             moe_supported(EK, EN, NE, NT, mx.Q8_0, "blk.0.ffn_gate_exps.weight"))]


def moe_forced_rows():
    return [
        ("MoE: F16 experts, MOE=1 -> offload", True, moe_supported(EK, EN, NE, NT, mx.F16, "blk.0.ffn_gate_exps.weight")),
        ("MoE: n_tokens=1, MOE=1 -> CPU", False, moe_supported(EK, EN, NE, 1, mx.Q8_0, "blk.1.ffn_gate_exps.weight")),
        ("MoE: F16 experts, src1 F16 declared -> offload", True,
         moe_supported(EK, EN, NE, NT, mx.F16, "blk.2.ffn_down_exps.weight", 4, PREC_F16)),
        ("MoE: F16 experts, src1 F32 declared -> CPU", False,
         moe_supported(EK, EN, NE, NT, mx.F16, "blk.3.ffn_down_exps.weight", 4, PREC_F32)),
    ]


def moe_src_admitted():
    """Four Q8_0 stacks of gpt-oss shape (4 experts each) in ONE weight buffer, budget 1.6x that
    buffer (test-rocket-placement.cpp:302-372): returns how many are admitted."""
    stack = EK * EN * 4 * 34 // 32
    buf_size = 4 * stack
    os.environ["MI355X_MOE_CACHE_MB"] = str((buf_size * 16 // 10) >> 20)
    buf_id = 0x7F0000001000
    n = 0
    for i in range(4):
        n += moe_supported(EK, EN, 4, 512, mx.Q8_0, f"blk.{i}.ffn_gate_exps.weight", 4, 0, (buf_id, buf_size))
    return n


def prec_quant_rows():
    # The reference's ROCKET_INT8 / ROCKET_INT4 select NPU integer routes that quantize the
    # activation; this backend has no such route (out of scope), so the knobs change nothing
    # and the declarations place as with the knobs unset.
    return [
        ("src1 F16 declared under INT8/INT4 -> offload (no integer route here)", True,
         mm_supported(256, 128, 256, mx.F16, 3, PREC_F16)),
        ("src1 Q8 declared -> offload", True, mm_supported(256, 128, 256, mx.F16, 3, PREC_Q8)),
        ("src1 Q4 declared -> offload", True, mm_supported(256, 128, 256, mx.F16, 3, PREC_Q4)),
        ("Q8_0 weight, src1 F16 declared -> offload", True, mm_supported(256, 128, 512, mx.Q8_0, 3, PREC_F16)),
    ]


def host_decoder_rows():
    """A quantized type the kernels do not decode is claimed once the plugin registers ggml's
    decoder for it (mi355x_backend_set_to_float), with ggml's block facts; bad registrations are
    refused and a natively decoded type keeps its device decoder."""
    def nop(src, dst, n):
        pass
    rows = [("Q4_1 leaf before registration -> CPU", False, mm_supported(256, 128, 512, mx.Q4_1))]
    st_bad_size = mx.set_to_float(mx.Q4_1, 32, 18, nop)        # Q4_1 blocks are 20 bytes
    st_bad_type = mx.set_to_float(70, 32, 18, nop)
    st_plain = mx.set_to_float(mx.F16, 1, 2, nop)
    st_native = mx.set_to_float(mx.Q4_K, 256, 144, nop)
    st_ok = mx.set_to_float(mx.Q4_1, 32, 20, nop)
    rows += [
        ("registration with wrong block bytes refused", True, st_bad_size == -1),
        ("registration of a type id past 63 refused", True, st_bad_type == -1),
        ("registration of a plain type refused", True, st_plain == -1),
        ("registration of a natively decoded type accepted and ignored", True, st_native == 0),
        ("registration of Q4_1 accepted", True, st_ok == 0),
        ("Q4_1 leaf, M >= quant floor -> offload", True, mm_supported(256, 128, 512, mx.Q4_1)),
        ("Q4_1 leaf, M(256) < quant floor -> CPU", False, mm_supported(256, 128, 256, mx.Q4_1)),
        ("Q4_1 leaf, K % 32 != 0 -> CPU", False, mm_supported(272, 128, 512, mx.Q4_1)),
        ("Q2_K leaf (not registered) -> CPU", False, mm_supported(256, 128, 512, mx.Q2_K)),
        ("Q4_1 expert stack (FORCED) -> offload", True, moe_supported(256, 128, 8, 512, mx.Q4_1, "blk.0.ffn_up_exps.weight")),
    ]
    return rows


if __name__ == "__main__":
    mode = sys.argv[1]
    fn = {"auto": moe_auto_rows, "budget": moe_budget_rows, "off": moe_off_rows, "forced": moe_forced_rows,
          "prec_quant": prec_quant_rows, "host_decoder": host_decoder_rows}.get(mode)
    if mode == "src_admitted":
        print(json.dumps(moe_src_admitted()))
    else:
        print(json.dumps([[a, bool(b), bool(c)] for a, b, c in fn()]))
