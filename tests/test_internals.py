"""Host-layer internals (CPU): the MB parser, weight identity, the circuit breaker, the fallback
counters and instance lifecycle -- test-rocket-internals.cpp's cases on this backend's API."""
import os

import numpy as np
import pytest

import ggml_mi355x as mx
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("text,ok,want", [
    ("0", True, 0), ("1", True, 1 << 20), (" 128 ", True, 128 << 20), ("", False, 12345),
    ("   ", False, 12345), ("-1", False, 12345), ("128junk", False, 12345), ("1e3", False, 12345),
    ("auto", False, 12345), (" auto ", False, 12345), ("99999999999999999999999", False, 12345),
])
def test_mb_parser(text, ok, want):
    """test-rocket-internals.cpp:78-104"""
    assert mx.parse_mb(text) == (ok, want)


def test_mb_parser_cap():
    assert mx.parse_mb("9223372036854775807") == (True, (1 << 40) << 20)


def _named(g, name, fill):
    t = g.new_tensor(mx.F32, [64, 16], name)
    g.set(t, (fill + 0.001 * np.arange(64 * 16)).astype(np.float32))
    return t


def test_weight_key_identity():
    """test-rocket-internals.cpp:108-150: the copy grammar, duplicate names, changed bytes."""
    g = mx.Graph()
    a, b = _named(g, "a#shared#0", 1.0), _named(g, "b#shared#1", 1.0)
    assert mx.weight_key(a) != mx.weight_key(b)
    assert mx.weight_key(a).startswith("a#shared#0@")
    orig = _named(g, "blk.0.attn_q.weight", 2.0)
    copy = _named(g, "MI355X#blk.0.attn_q.weight#0", 2.0)
    assert mx.weight_key(orig) == mx.weight_key(copy)
    trunc = _named(g, "MI355X#blk.0.attn_q.weight", 2.0)
    assert mx.weight_key(trunc) == mx.weight_key(orig)
    other_backend = _named(g, "ROCKET#blk.0.attn_q.weight#0", 2.0)
    assert mx.weight_key(other_backend) != mx.weight_key(orig)   # only this backend's grammar
    same = _named(g, "blk.0.attn_q.weight", 3.0)
    assert mx.weight_key(same) != mx.weight_key(orig)
    before = mx.weight_key(orig)
    assert mx.weight_key(orig) == before
    arr = g.get(orig, np.float32, (16, 64))
    arr[0, 0] += 1.0
    g.set(orig, arr)
    assert mx.weight_key(orig) != before
    assert mx.weight_key(_named(g, "leaf_12", 1.0)) == ""
    assert mx.weight_key(_named(g, "node_7", 1.0)) == ""
    assert mx.weight_key(_named(g, "leaf_", 1.0)).startswith("leaf_@")
    nd = mx.Graph(alloc=False).new_tensor(mx.F32, [64, 16], "blk.3.ffn_up.weight")
    assert mx.weight_key(nd) == "blk.3.ffn_up.weight"


def _tiny_mm(g):
    K, N, M = 64, 64, 32
    W = g.new_tensor(mx.F16, [K, N], "blk.0.tiny.weight")
    X = g.new_tensor(mx.F32, [K, M])
    g.set(W, O.f32_to_f16_bits(O.fill_uniform((N, K), 1, 1.0)))
    g.set(X, O.fill_uniform((M, K), 2, 1.0))
    return W, X, g.mul_mat(W, X)


def test_breaker_transitions():
    """test-rocket-internals.cpp:535-561, end to end: device failures forced from the host.
    Three consecutive failures open the route for 64 calls, a failed probe reopens it for 128,
    and every op still produces the CPU fallback's result."""
    be = mx.Backend()
    g = mx.Graph()
    W, X, d = _tiny_mm(g)
    be.inject_faults("gemm", 10000)
    want = O.mul_mat(O.F16, g.get(W, np.uint16, (64, 64)), g.get(X, np.float32, (32, 64)), 64, 64)
    for i in range(3):
        assert be.compute([d]) == mx.STATUS_SUCCESS
    assert be.route_stats("gemm") == (3, 3, 0)
    for i in range(64):
        be.compute([d])
    assert be.route_stats("gemm") == (3, 3, 64)           # open: no device attempt
    be.compute([d])
    assert be.route_stats("gemm") == (4, 4, 64)           # the probe, failed
    for i in range(128):
        be.compute([d])
    assert be.route_stats("gemm") == (4, 4, 192)          # reopened for twice as long
    assert be.cpu_fallbacks() == 3 + 64 + 1 + 128
    assert be.route_ops("mt") + be.route_ops("prepacked") == 196
    got = g.get(d, np.float32, (32, 64))
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    be.free()


def test_instance_lifecycle():
    L = mx.host()
    a, b = mx.Backend(), mx.Backend()
    assert L.mi355x_backend_is(a.h) and L.mi355x_backend_is(b.h)
    assert L.mi355x_backend_get_n_threads(a.h) == 5
    L.mi355x_backend_set_n_threads(a.h, 12)
    assert L.mi355x_backend_get_n_threads(a.h) == 8        # clamped
    L.mi355x_backend_set_n_threads(a.h, 3)
    assert L.mi355x_backend_get_n_threads(a.h) == 3
    assert a.route_ops() == 0 and a.cpu_fallbacks() == 0 and a.moe_stats() == (0, 0)
    assert L.mi355x_backend_name() == b"MI355X"
    a.free()
    b.free()


def test_unknown_op_fails_graph():
    be = mx.Backend()
    g = mx.Graph()
    A = g.new_tensor(mx.F32, [8, 8])
    add = g.op(mx.F32, [8, 8], mx.OP_ADD, (A, A))
    assert be.compute([add]) == mx.STATUS_FAILED
    view = g.permute_view(A, [8, 8, 1, 1], [4, 32, 256, 256])
    assert be.compute([view]) == mx.STATUS_SUCCESS
    be.free()


def test_moe_bad_id_fails_graph():
    """An id outside [0, n_expert) is a malformed graph (ggml-rocket.cpp:6719)."""
    be = mx.Backend()
    g = mx.Graph()
    K, N, E, U, T = 64, 64, 4, 2, 8
    a = g.new_tensor(mx.F16, [K, N, E], "blk.0.ffn_up_exps.weight")
    b = g.new_tensor(mx.F32, [K, 1, T])
    ids = g.new_tensor(mx.I32, [U, T])
    idv = np.zeros((T, U), np.int32)
    idv[5, 1] = E
    g.set(ids, idv)
    assert be.compute([g.mul_mat_id(a, b, ids)]) == mx.STATUS_FAILED
    be.free()


def test_expert_ledger_across_backends(tmp_path):
    """test-rocket-internals.cpp:155-215: the expert-stack ledger with several live backends
    (placement's spare copy, a second backend's own copy, a refused copy, copies returned on
    free, the ledger forgotten with the last backend). The ledger has no ABI entry, so a small
    C++ program links the host sources and calls it directly."""
    import subprocess
    root = os.path.dirname(HERE)
    host = os.path.join(root, "ggml-rocket_amd", "csrc", "host")
    exe = str(tmp_path / "ledger_test")
    cmd = ["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           os.path.join(HERE, "cpp", "ledger_test.cpp"), os.path.join(host, "claims.cpp"),
           os.path.join(host, "knobs.cpp"), "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib",
           "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True)
    env = {k: v for k, v in os.environ.items() if not k.startswith(("MI355X_", "ROCKET_"))}
    env["HIP_VISIBLE_DEVICES"] = ""
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
