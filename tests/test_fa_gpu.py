"""FLASH_ATTN_EXT on the GPU against the double oracle, through the C ABI.

The reference's cases (test-rocket-fa.cpp): overflow (one-hot softmax, raw q.k past 65504),
typical (random, causal), scaled (scaled logits past 65504) and q range (scaled Q past 65504).
The reference sends the last two to its host fallback because its NPU keeps an fp16 score
surface; here scores stay in fp32 registers and a Q row past fp16 range is divided by a per-row
factor, so all four run on the device, scored against the same oracle and tolerances.
Plus the prefill attention shapes: 32 query / 8 KV heads, d 128, 512 tokens, n_kv 1024/4096/8192,
N(0,1) inputs, causal mask, scale 1/sqrt(128); scored on sampled query rows. Every case runs
under both block layouts (two or four wave tasks per block).
"""
import numpy as np
import pytest

from oracle import oracle as O
from fa_cases import REFERENCE_CASES, fill_case, causal_mask, TYPICAL, SCALED, QRANGE
from bars import compare

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[2, 4], ids=["tasks2", "tasks4"], autouse=True)
def fa_tasks(request, monkeypatch):
    """Every case under both block layouts: two wave tasks per block (four waves a task, each
    taking one 32-key half of alternate tiles) and four (two waves a task). The library picks
    between them per call; MI355X_FA_TASKS pins the choice (builds with DV 256 have only four)."""
    monkeypatch.setenv("MI355X_FA_TASKS", str(request.param))
    return request.param


@pytest.fixture(scope="module")
def mx(torch_cuda):
    import ggml_mi355x
    ggml_mi355x.lib()
    return ggml_mi355x


def _run(mx, Q, K16, V16, M16, scale, softcap=0.0, nsplit=0):
    import torch
    q = torch.from_numpy(Q).cuda()
    k = torch.from_numpy(K16.view(np.float16)).cuda()
    v = torch.from_numpy(V16.view(np.float16)).cuda()
    m = torch.from_numpy(M16.view(np.float16)).cuda() if M16 is not None else None
    out = mx.flash_attn(q, k, v, m, scale, softcap=softcap, nsplit=nsplit)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("case", REFERENCE_CASES, ids=[c[0] for c in REFERENCE_CASES])
@pytest.mark.parametrize("nsplit", [1, 0])
def test_fa_reference_cases(mx, case, nsplit):
    name, D, T, H, KV, HK, kind, tol = case
    Q, K, V, M = fill_case(D, T, H, KV, HK, kind)
    K16, V16, M16 = O.f32_to_f16_bits(K), O.f32_to_f16_bits(V), O.f32_to_f16_bits(M)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    q_mode = 1 if kind in (SCALED, QRANGE) else 0
    want = O.flash_attn(Q, K16, V16, M16, scale, q_mode=q_mode)
    got = _run(mx, Q, K16, V16, M16, scale, nsplit=nsplit)
    assert np.isfinite(got).all(), name
    err = float(np.abs(got.astype(np.float64) - want).max())
    print(f"{name} nsplit={nsplit}: max abs err {err:.3g} (tol {tol})")
    assert err <= tol, name


def test_fa_fully_masked_rows_are_zero(mx):
    """A row whose every key is masked is written as zeros (ggml-rocket.cpp:5395-5397)."""
    D, T, H, KV, HK = 64, 40, 4, 300, 2
    Q, K, V, _ = fill_case(D, T, H, KV, HK, TYPICAL)
    M = causal_mask(T, KV)
    M[5, :] = -np.inf
    M[33, :] = -np.inf
    K16, V16, M16 = O.f32_to_f16_bits(K), O.f32_to_f16_bits(V), O.f32_to_f16_bits(M)
    for ns in (1, 3):
        got = _run(mx, Q, K16, V16, M16, 0.125, nsplit=ns)
        assert np.all(got[5] == 0.0) and np.all(got[33] == 0.0)
        want = O.flash_attn(Q, K16, V16, M16, 0.125)
        assert float(np.abs(got - want).max()) <= 2e-2


def test_fa_softcap_unmasked_ragged(mx):
    """Soft-cap, no mask, and T / KV that are not multiples of the tiles."""
    D, T, H, KV, HK = 128, 45, 6, 333, 3
    Q = O.fill_normal((H, T, D), 901)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 902))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 903))
    scale = 0.3
    for softcap in (0.0, 5.0):
        want = O.flash_attn(Q, K16, V16, None, scale, softcap=softcap)
        for ns in (1, 2):
            got = _run(mx, Q, K16, V16, None, scale, softcap=softcap, nsplit=ns)
            r = compare(want, got)
            assert r["nonfinite"] == 0 and r["range_err"] <= 1e-2, (softcap, ns, r)


def test_fa_strided_views(mx):
    """Q as a permuted [T][H][D] buffer and K/V as KV-cache slices [KV][HK][D] (llama.cpp's
    layouts), read in place through the strides."""
    import torch
    import ggml_mi355x as mxm
    D, T, H, KV, HK = 128, 64, 8, 512, 2
    Qthd = O.fill_normal((T, H, D), 911)
    Kc = O.f32_to_f16_bits(O.fill_normal((KV, HK, D), 912))
    Vc = O.f32_to_f16_bits(O.fill_normal((KV, HK, D), 913))
    M = causal_mask(T, KV)
    q = torch.from_numpy(Qthd).cuda().permute(1, 0, 2)           # [H][T][D] view
    k = torch.from_numpy(Kc.view(np.float16)).cuda().permute(1, 0, 2)
    v = torch.from_numpy(Vc.view(np.float16)).cuda().permute(1, 0, 2)
    m = torch.from_numpy(O.f32_to_f16_bits(M).view(np.float16)).cuda()
    got = mxm.flash_attn(q, k, v, m, 0.088)
    torch.cuda.synchronize()
    want = O.flash_attn(np.ascontiguousarray(Qthd.transpose(1, 0, 2)),
                        np.ascontiguousarray(Kc.transpose(1, 0, 2)),
                        np.ascontiguousarray(Vc.transpose(1, 0, 2)), O.f32_to_f16_bits(M), 0.088)
    r = compare(want, got.cpu().numpy())
    assert r["nonfinite"] == 0 and r["range_err"] <= 1e-2, r


@pytest.mark.parametrize("KV", [1024, 4096, 8192])
def test_fa_baseline_shapes(mx, KV):
    """32 query heads, 8 KV heads, d 128, 512 tokens; K/V ~N(0,1) fp16; causal F16 mask;
    scale 1/sqrt(128). Scored on 48 sampled tokens (all heads) against the double oracle."""
    D, T, H, HK = 128, 512, 32, 8
    Q = O.fill_normal((H, T, D), 0x5EED0000 + 48)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 0x5EED0000 + 49))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 0x5EED0000 + 50))
    M16 = O.f32_to_f16_bits(causal_mask(T, KV))
    scale = float(1.0 / np.sqrt(128.0))
    got = _run(mx, Q, K16, V16, M16, scale)
    rows = np.unique(np.linspace(0, T - 1, 48).astype(int))
    want = O.flash_attn(np.ascontiguousarray(Q[:, rows, :]), K16, V16,
                        np.ascontiguousarray(M16[rows]), scale)
    r = compare(want, got[rows])
    print(f"FA KV={KV}: max abs {r['max_abs']:.3g} range_err {r['range_err']:.3g}")
    assert r["nonfinite"] == 0
    assert r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2


@pytest.mark.parametrize("H,HK", [(3, 3), (6, 3), (8, 2)])
def test_fa_mask_holes_and_skipped_tiles(mx, H, HK):
    """A mask with scattered -inf entries, a 128-key band masked for every query (whole key tiles
    skipped inside the visible range), fully masked rows, and a tail masked for the first query
    tile only; GQA groups of 1, 2 and 4 (a block's waves on different query tiles when < 4)."""
    D, T, KV = 64, 96, 640
    Q = O.fill_normal((H, T, D), 940)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 941))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 942))
    rnd = O.fill_uniform((T, KV), 943, 1.0)
    M = np.where(rnd > 0.4, -np.inf, 0.0).astype(np.float32)
    M[:, 128:256] = -np.inf
    M[40:48, :] = -np.inf
    M[:32, 576:] = -np.inf
    M16 = O.f32_to_f16_bits(M)
    want = O.flash_attn(Q, K16, V16, M16, 0.125)
    for ns in (1, 2, 5):
        got = _run(mx, Q, K16, V16, M16, 0.125, nsplit=ns)
        assert np.all(got[40:48] == 0.0), ns
        r = compare(want, got)
        assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2, (ns, r)


@pytest.mark.parametrize("H,HK,softcap", [(16, 2, 0.0), (8, 8, 0.0), (16, 2, 30.0)])
def test_fa_mla_k192_v128(mx, H, HK, softcap):
    """Keys of 192 and values of 128 (DeepSeek-style MLA heads after decompression): causal
    mask with scattered holes and a fully masked row, a ragged n_kv under a padded mask row,
    GQA groups of 8 and 1, softcap; split-K off, on, and chosen by the library."""
    D, DV, T, KV = 192, 128, 96, 601
    Q = O.fill_normal((H, T, D), 950)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 951))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, DV), 952))
    # mask rows padded to 608 halves as ggml pads them; the columns past n_kv are never read
    M = np.full((T, 608), 7.0, np.float32)
    M[:, :KV] = causal_mask(T, KV)
    rnd = O.fill_uniform((T, KV), 953, 1.0)
    M[:, :KV][rnd > 0.7] = -np.inf
    M[17, :] = -np.inf
    M16 = O.f32_to_f16_bits(M)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = O.flash_attn(Q, K16, V16, M16, scale, softcap=softcap)
    for ns in (1, 2, 0):
        got = _run(mx, Q, K16, V16, M16, scale, softcap=softcap, nsplit=ns)
        assert got.shape == (T, H, DV)
        assert np.all(got[17] == 0.0), ns
        r = compare(want, got)
        print(f"MLA H={H} HK={HK} softcap={softcap} nsplit={ns}: {r}")
        assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2, (ns, r)


@pytest.mark.parametrize("D,DV,softcap", [(32, 32, 0.0), (96, 96, 0.0), (128, 64, 0.0), (64, 128, 0.0),
                                          (160, 80, 0.0), (192, 64, 0.0), (256, 256, 0.0), (256, 256, 50.0),
                                          (192, 192, 0.0), (224, 160, 0.0)])
def test_fa_padded_head_dims(mx, D, DV, softcap):
    """Head dims between the built kernels (64/64, 128/128, 192/128, 256/256; the last with one
    wave per query tile) run zero-padded onto the
    smallest that holds them: Q and K columns past dk and V columns past dv read as zero, output
    columns past dv are not written (checked on a NaN-filled output with a row stride wider than
    dv). Causal mask with holes and a fully masked row, GQA 4:1, ragged T and n_kv; split-K off,
    on, and chosen by the library."""
    import torch
    H, HK, T, KV = 8, 2, 70, 389
    Q = O.fill_normal((H, T, D), 990 + D)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 991 + D))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, DV), 992 + DV))
    M = np.full((T, 392), 7.0, np.float32)
    M[:, :KV] = causal_mask(T, KV)
    rnd = O.fill_uniform((T, KV), 993, 1.0)
    M[:, :KV][rnd > 0.8] = -np.inf
    M[5, :] = -np.inf
    M16 = O.f32_to_f16_bits(M)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = O.flash_attn(Q, K16, V16, M16, scale, softcap=softcap)
    q = torch.from_numpy(Q).cuda()
    k = torch.from_numpy(K16.view(np.float16)).cuda()
    v = torch.from_numpy(V16.view(np.float16)).cuda()
    m = torch.from_numpy(M16.view(np.float16)).cuda()
    for ns in (1, 3, 0):
        wide = torch.full((T, H, DV + 16), float("nan"), dtype=torch.float32, device="cuda")
        out = wide[:, :, :DV]
        mx.flash_attn(q, k, v, m, scale, softcap=softcap, nsplit=ns, out=out)
        torch.cuda.synchronize()
        w = wide.cpu().numpy()
        assert np.isnan(w[:, :, DV:]).all(), ("wrote past dv", ns)
        got = w[:, :, :DV]
        assert np.all(got[5] == 0.0), ns
        r = compare(want, got)
        print(f"padded D={D} DV={DV} softcap={softcap} nsplit={ns}: {r}")
        assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2, (ns, r)


@pytest.mark.parametrize("D,DV,H,HK,softcap", [(576, 512, 16, 1, 0.0), (576, 512, 8, 1, 30.0), (320, 264, 8, 2, 0.0),
                                               (288, 128, 8, 4, 0.0), (128, 512, 4, 1, 0.0)])
def test_fa_wide_head_dims(mx, D, DV, H, HK, softcap):
    """Head dims past 256 (the absorbed MLA's 576 / 512, and any dk % 32 == 0, dv % 8 == 0 up to
    1024) run as two GEMMs around a softmax pass: causal mask with holes and a fully masked row,
    ragged T and n_kv, output columns past dv untouched (NaN-filled output with a wider row)."""
    import torch
    T, KV = 70, 389
    Q = O.fill_normal((H, T, D), 1990 + D)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 1991 + D))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, DV), 1992 + DV))
    M = np.full((T, 392), 7.0, np.float32)
    M[:, :KV] = causal_mask(T, KV)
    rnd = O.fill_uniform((T, KV), 1993, 1.0)
    M[:, :KV][rnd > 0.8] = -np.inf
    M[5, :] = -np.inf
    M16 = O.f32_to_f16_bits(M)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = O.flash_attn(Q, K16, V16, M16, scale, softcap=softcap)
    q = torch.from_numpy(Q).cuda()
    k = torch.from_numpy(K16.view(np.float16)).cuda()
    v = torch.from_numpy(V16.view(np.float16)).cuda()
    m = torch.from_numpy(M16.view(np.float16)).cuda()
    wide = torch.full((T, H, DV + 16), float("nan"), dtype=torch.float32, device="cuda")
    out = wide[:, :, :DV]
    mx.flash_attn(q, k, v, m, scale, softcap=softcap, out=out)
    torch.cuda.synchronize()
    w = wide.cpu().numpy()
    assert np.isnan(w[:, :, DV:]).all(), "wrote past dv"
    got = w[:, :, :DV]
    assert np.all(got[5] == 0.0)
    r = compare(want, got)
    print(f"wide D={D} DV={DV} H={H} HK={HK} softcap={softcap}: {r}")
    assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2, r


def test_fa_wide_mla_prefill_chunked(mx):
    """The absorbed-MLA shape at prefill size, 16 query heads on one KV head, 512 queries over 4100
    keys (causal, last 512 positions): the 8192 query rows take three chunks of the scores'
    workspace slab; sampled tokens against the oracle."""
    import torch
    H, HK, T, KV, D, DV = 16, 1, 512, 4100, 576, 512
    Q = O.fill_normal((H, T, D), 2990)
    K16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, D), 2991))
    V16 = O.f32_to_f16_bits(O.fill_normal((HK, KV, DV), 2992))
    M = causal_mask(T, KV)
    M16 = O.f32_to_f16_bits(M)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    q = torch.from_numpy(Q).cuda()
    k = torch.from_numpy(K16.view(np.float16)).cuda()
    v = torch.from_numpy(V16.view(np.float16)).cuda()
    m = torch.from_numpy(M16.view(np.float16)).cuda()
    got = mx.flash_attn(q, k, v, m, scale).cpu().numpy()
    idx = np.array([0, 1, 137, 255, 256, 400, 510, 511])
    want = O.flash_attn(np.ascontiguousarray(Q[:, idx, :]), K16, V16, np.ascontiguousarray(M16[idx, :]), scale)
    r = compare(want, got[idx])
    print(f"wide MLA prefill sampled rows: {r}")
    assert r["nonfinite"] == 0 and r["max_abs"] <= 2e-2 and r["range_err"] <= 1e-2, r


@pytest.mark.parametrize("nsplit", [1, 3])
def test_fa_classes_ready_reuses_the_mask_classes(mx, nsplit):
    """mi355x_flash_attn_ex with MI355X_FA_CLASSES_READY: the layers of a micro-batch share one
    mask, so the first call classifies its tiles into the workspace and later calls with other
    Q / K / V skip that pass. Each reusing call gives the same bits as a call that classifies the
    mask itself, with a causal mask holding all three tile classes and a fully masked row, split
    and unsplit; the first call's own result matches the oracle."""
    import torch
    D, T, H, KV, HK = 128, 200, 8, 700, 2
    M = causal_mask(T, KV)
    M[17, :] = -np.inf
    M16 = O.f32_to_f16_bits(M)
    m = torch.from_numpy(M16.view(np.float16)).cuda()
    scale = 1.0 / np.sqrt(D)
    ws = None
    for layer in range(3):
        Q = O.fill_normal((H, T, D), 0x9100 + layer)
        K, V = O.fill_normal((HK, KV, D), 0x9110 + layer), O.fill_normal((HK, KV, D), 0x9120 + layer)
        K16, V16 = O.f32_to_f16_bits(K), O.f32_to_f16_bits(V)
        q = torch.from_numpy(np.ascontiguousarray(Q)).cuda()
        k = torch.from_numpy(K16.view(np.float16)).cuda()
        v = torch.from_numpy(V16.view(np.float16)).cuda()
        if ws is None:
            ws = torch.empty(mx.flash_attn_workspace(q, k, v, m, torch.empty((T, H, D), device="cuda"), scale,
                                                     nsplit=nsplit), dtype=torch.uint8, device="cuda")
        fresh = mx.flash_attn(q, k, v, m, scale, nsplit=nsplit).cpu().numpy()
        got = mx.flash_attn(q, k, v, m, scale, nsplit=nsplit, workspace=ws, classes_ready=layer > 0)
        torch.cuda.synchronize()
        got = got.cpu().numpy()
        assert np.array_equal(got, fresh), (layer, nsplit)
        if layer == 0:
            want = O.flash_attn(Q, K16, V16, M16, scale)
            assert np.all(got[17] == 0.0) and float(np.abs(got - want).max()) <= 2e-2
