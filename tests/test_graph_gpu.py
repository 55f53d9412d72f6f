"""HIP-graph capture of the device entries: a captured call replayed several times, with eager
work between the replays (new inputs copied in, the output poisoned with NaN), must give on every
replay what the eager call gives for the same inputs. Covers the skinny GEMM with a K split (its
output cleared by the activation pack kernel inside the graph, no memset node) and attention
with a KV split and its merge pass."""
import math

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx(torch_cuda):
    import ggml_mi355x
    ggml_mi355x.lib()
    return ggml_mi355x


def _capture(fn):
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def test_graph_skinny_mul_mat_k_split(mx):
    import torch
    M, N, K = 32, 400, 2560
    W = O.fill_normal((N, K), 1200, 0.0, 0.02)
    w = mx.upload_weight(O.Q4_K, O.quantize(O.Q4_K, W), N, K)
    x = torch.empty((M, K), dtype=torch.float32, device="cuda")
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ws = torch.empty(int(mx.lib().mi355x_mul_mat_workspace_for(O.Q4_K, N, K, M)), dtype=torch.uint8, device="cuda")
    inputs = [torch.from_numpy(O.fill_normal((M, K), 1201 + i)).cuda() for i in range(3)]
    refs = []
    for X in inputs:
        x.copy_(X)
        mx.mul_mat(O.Q4_K, w, N, K, x, out, ws)
        torch.cuda.synchronize()
        refs.append(out.clone())
    g = _capture(lambda: mx.mul_mat(O.Q4_K, w, N, K, x, out, ws))
    for rep in range(2):
        for i, (X, ref) in enumerate(zip(inputs, refs)):
            x.copy_(X)
            out.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            want = ref.cpu().numpy()
            assert np.isfinite(got).all(), (rep, i)
            # the K-split partials are summed in split order: every replay gives the eager bits
            assert np.array_equal(got, want), (rep, i)


def test_graph_flash_attn_kv_split(mx):
    import torch
    T, H, HK, D, KV = 64, 8, 2, 128, 1500
    q = torch.empty((H, T, D), dtype=torch.float32, device="cuda")
    k = torch.from_numpy(O.fill_normal((HK, KV, D), 1211)).cuda().half()
    v = torch.from_numpy(O.fill_normal((HK, KV, D), 1212)).cuda().half()
    j = torch.arange(KV, device="cuda")[None, :]
    t = torch.arange(T, device="cuda")[:, None]
    m = torch.where(j > KV - T + t, float("-inf"), 0.0).half()
    out = torch.empty((T, H, D), dtype=torch.float32, device="cuda")
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    scale = 1.0 / math.sqrt(D)
    inputs = [torch.from_numpy(O.fill_normal((H, T, D), 1213 + i)).cuda() for i in range(3)]
    refs = []
    for X in inputs:
        q.copy_(X)
        mx.flash_attn(q, k, v, m, scale, nsplit=3, out=out, workspace=ws)
        torch.cuda.synchronize()
        refs.append(out.clone())
    g = _capture(lambda: mx.flash_attn(q, k, v, m, scale, nsplit=3, out=out, workspace=ws))
    for rep in range(2):
        for i, (X, ref) in enumerate(zip(inputs, refs)):
            q.copy_(X)
            out.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref), (rep, i)
