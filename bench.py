#!/usr/bin/env python3
"""Prefill benchmark: the backend-claimed ops of an 8B-shape Q4_K prefill on one MI355X.

Workload (metric "prefill tok/s (8B-shape Q4_K, 2048 tok)"): a Llama-3-8B-shaped stack
(32 layers, d 4096, FFN 14336, 32 query / 8 KV heads, head dim 128) with random-init Q4_K
weights (quantized from N(0, 0.02); every layer distinct), prefilling 2048 tokens in 4
micro-batches of 512. One step runs, per micro-batch and layer, exactly the ops this backend
claims in such a prefill under its default knobs: the fused Q/K/V projection group,
FLASH_ATTN_EXT over the causal KV prefix where n_kv >= FLASH_ATTN_MIN_KV (1024: micro-batches 2-4,
n_kv 1024 / 1536 / 2048; the first micro-batch's n_kv 512 attention is declined and runs on the
host's CPU backend), the output projection, the fused gate/up group and the down projection.
Ops the backend never claims (norms, RoPE, SiLU-mul, residual adds, the last-token lm_head at
M=1) are not in the step, so `value` is the rate of the backend's share of the prefill with its
inputs resident in HBM, not an end-to-end prefill rate; the rate through the plugin boundary with
host buffers (PCIe-inclusive) is reported beside it under "host_path".

Routes: "prepacked-q" (default; the reference's ROCKET_QUANT_RESIDENT route): each Q4_K weight
is decoded once to an fp16 HBM copy and the GEMMs read fp16. "mt": the GEMMs read the Q4_K
blocks and dequantize them in LDS on every call (the backend's mt route instead decodes the
smaller panels, qkv and o, to fp16 scratch first where mi355x_mul_mat_decode_first says so; this
step keeps the in-GEMM decode for all four).

Prints ONE JSON line (rank 0). `value` is tokens/s of the whole step; `roofline` is the dominant
kernel's (the GEMM) live HIP-event figure; `cpu_baseline` is the CPU oracle timed on a bounded
sample of the same workload on this host.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "ggml-rocket_amd"))

METRIC = "prefill tok/s (8B-shape Q4_K, 2048 tok); MUL_MAT/FA TFLOP/s vs MFMA peak"
PEAK_F16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# HBM bytes per GEMM launch (mean of a layer's four launches at M = 512, fp16-resident route),
# from rocprofv3 FETCH_SIZE / WRITE_SIZE runs of `bench.py --pmc-probe` scaled by a plain copy's
# reading. Counters cannot be read inside the timed run, so the figure comes from the committed
# profile, which records the SHA-256 of the GEMM source it was measured on: when the source has
# changed since, the figure is stale and `traffic` is reported as null.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "prefill_8b_hbm_traffic_pmc.md")
GEMM_SOURCE = os.path.join(ROOT, "ggml-rocket_amd", "csrc", "mx_gemm.hip")


def gemm_traffic(route):
    """(bytes per GEMM launch, provenance) from the traffic profile, or (None, reason)."""
    import hashlib
    import re
    if route != "prepacked-q":
        return None, "not measured for this route"
    try:
        text = open(TRAFFIC_PROFILE).read()
        src = hashlib.sha256(open(GEMM_SOURCE, "rb").read()).hexdigest()
    except OSError as exc:
        return None, f"unavailable ({exc.__class__.__name__})"
    m = re.search(r"traffic_bytes_per_gemm_launch:\s*([0-9.eE+]+)\s+mx_gemm\.hip sha256:\s*([0-9a-f]{64})", text)
    if not m:
        return None, "no machine-readable line in the profile"
    if m.group(2) != src:
        return None, "stale: mx_gemm.hip changed since the profile was measured"
    return float(m.group(1)), "profiles/prefill_8b_hbm_traffic_pmc.md (source hash matches)"


L_LAYERS, D_MODEL, FFN, NH, NKV, HD = 32, 4096, 14336, 32, 8, 128
TOKENS, UBATCH = 2048, 512


def synth_q4k(N, K, seed, sigma=0.02):
    """Synthetic workload weights: an [N, K] matrix drawn from N(0, sigma) and quantized to ggml's
    Q4_K blocks (144 bytes per 256 weights: fp16 d, fp16 dmin, 12 bytes of packed 6-bit
    sub-block scales and mins, 128 bytes of nibbles). A plain min/max quantizer: every sub-block
    of 32 spans [min(0, lo), hi] in 15 steps, the block's d / dmin are the largest sub-block
    scale / min over 63. Returns the payload as flat uint8."""
    import numpy as np
    rng = np.random.default_rng(seed)
    out = np.empty((N, K // 256, 144), dtype=np.uint8)
    for r0 in range(0, N, 512):   # row chunks keep the temporaries cache-sized
        n = min(512, N - r0)
        B = (rng.standard_normal((n, K), dtype=np.float32) * np.float32(sigma)).reshape(n, K // 256, 8, 32)
        lo = np.minimum(B.min(axis=3), np.float32(0))
        sub_scale = (B.max(axis=3) - lo) * np.float32(1 / 15)
        sub_min = -lo
        d = (sub_scale.max(axis=2) * np.float32(1 / 63)).astype(np.float16)
        dmin = (sub_min.max(axis=2) * np.float32(1 / 63)).astype(np.float16)
        df = np.maximum(d.astype(np.float32), np.float32(1e-30))[..., None]
        dmf = np.maximum(dmin.astype(np.float32), np.float32(1e-30))[..., None]
        sc = np.clip(np.rint(sub_scale / df), 0, 63).astype(np.uint8)
        mn = np.clip(np.rint(sub_min / dmf), 0, 63).astype(np.uint8)
        step = np.maximum(df * sc, np.float32(1e-30))[..., None]
        q = np.clip(np.rint((B + (dmf * mn)[..., None]) / step), 0, 15).astype(np.uint8)
        o = out[r0:r0 + n]
        o[..., 0:2] = d[..., None].view(np.uint8)
        o[..., 2:4] = dmin[..., None].view(np.uint8)
        o[..., 4:8] = sc[..., :4] | ((sc[..., 4:] >> 4) << 6)
        o[..., 8:12] = mn[..., :4] | ((mn[..., 4:] >> 4) << 6)
        o[..., 12:16] = (sc[..., 4:] & 15) | ((mn[..., 4:] & 15) << 4)
        q = q.reshape(n, K // 256, 4, 2, 32)   # (64-weight group, low / high nibble, 32)
        o[..., 16:] = (q[..., 0, :] | (q[..., 1, :] << 4)).reshape(n, K // 256, 128)
    return out.reshape(-1)

def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--route", choices=["prepacked-q", "mt"], default="prepacked-q")
    p.add_argument("--layers", type=int, default=L_LAYERS)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=0,
                   help="threads of the CPU baseline (default: OMP_NUM_THREADS, else every core this "
                        "process may run on)")
    p.add_argument("--fa-min-kv", type=int, default=1024,
                   help="FLASH_ATTN_EXT runs in the step where n_kv >= this (the backend's default claim)")
    p.add_argument("--quick", action="store_true",
                   help="only the step and its roofline: no CPU baseline, single-op configurations "
                        "or host-path run")
    p.add_argument("--host-path", action="store_true",
                   help="run the prefill through graph_compute with host tensors (the plugin "
                        "boundary, PCIe-inclusive) and print that rate instead")
    p.add_argument("--gguf", default=None,
                   help="with --host-path: take the model (dims, tensor names, weight bytes) from this "
                        "llama GGUF, memory-mapped (e.g. one written by ggml-rocket_amd/llama3_gguf.py)")
    p.add_argument("--configs", action="store_true",
                   help="time the single-op configurations (F16 MUL_MAT 8192x2048 at M 512; Q8_0 / Q4_K / "
                        "Q6_K MUL_MAT at K,N in {3072x3072, 3072x8192, 8192x3072}, M in {32, 128, 512, "
                        "2048}; FLASH_ATTN_EXT 32/8 heads, d 128, 512 queries, n_kv 1024/4096/8192) against "
                        "their rooflines and print one JSON line")
    p.add_argument("--moe", action="store_true",
                   help="time MUL_MAT_ID at the 128-expert / top-8 / 512-token / d 2048 / FFN 768 Q4_K "
                        "shape (gate/up and down, cold expert stacks) and print one JSON line")
    p.add_argument("--mul-mat", default=None, metavar="TYPE,N,K,M",
                   help="time one single-op MUL_MAT (e.g. Q4_K,8192,3072,128) through mi355x_mul_mat as the "
                        "--configs sweep does, 64 replayed calls, and print one JSON line (for kernel traces "
                        "of one shape)")
    p.add_argument("--pmc-probe", action="store_true",
                   help="for hardware-counter runs: launch each distinct op of one layer once, "
                        "eagerly, then a plain 1 GiB device copy (the calibration kernel), and exit")
    return p.parse_args()


class Prefill:
    def __init__(self, route, n_layers, fa_min_kv=1024):
        import numpy as np
        import torch
        import ggml_mi355x as mx
        self.mx, self.torch, self.np = mx, torch, np
        self.route = route
        self.fa_min_kv = fa_min_kv
        self.wt = mx.F16_T if route == "prepacked-q" else mx.Q4_K
        dev = "cuda"
        t0 = time.time()
        shapes = {"q": (D_MODEL, D_MODEL), "k": (NKV * HD, D_MODEL), "v": (NKV * HD, D_MODEL),
                  "o": (D_MODEL, D_MODEL), "gate": (FFN, D_MODEL), "up": (FFN, D_MODEL),
                  "down": (D_MODEL, FFN)}
        self.shapes = shapes
        # layer 0: quantized on the host from N(0, 0.02); the other layers get fresh random
        # nibbles under layer 0's block headers (valid Q4_K, distinct bytes per layer)
        self.host_q4 = {}
        base = {}
        for i, (name, (N, K)) in enumerate(shapes.items()):
            self.host_q4[name] = synth_q4k(N, K, 0x5EED0000 + 80 + i)
            base[name] = torch.from_numpy(self.host_q4[name]).to(dev)
        g = torch.Generator(device=dev)
        g.manual_seed(1234)
        self.layers = []
        for li in range(n_layers):
            lw = {}
            for name, (N, K) in shapes.items():
                q = base[name].clone() if li == 0 else base[name].clone()
                if li > 0:
                    blk = q.view(-1, 144)
                    blk[:, 16:] = torch.randint(0, 256, (blk.shape[0], 128), dtype=torch.uint8, device=dev,
                                                generator=g)
                if self.wt == mx.F16_T:
                    lw[name] = mx.tile_f16(mx.Q4_K, q, N, K)
                    del q
                else:
                    lw[name] = q
            self.layers.append(lw)
        torch.cuda.synchronize()
        self.setup_s = time.time() - t0
        # activations / scratch
        f32 = torch.float32
        T = UBATCH
        self.x = torch.randn(T, D_MODEL, device=dev, dtype=f32)
        self.qo = torch.empty(T, D_MODEL, device=dev, dtype=f32)
        self.ko = torch.empty(T, NKV * HD, device=dev, dtype=f32)
        self.vo = torch.empty(T, NKV * HD, device=dev, dtype=f32)
        self.attn = torch.empty(T, NH * HD, device=dev, dtype=f32)
        self.oo = torch.empty(T, D_MODEL, device=dev, dtype=f32)
        self.go = torch.empty(T, FFN, device=dev, dtype=f32)
        self.uo = torch.empty(T, FFN, device=dev, dtype=f32)
        self.act = torch.randn(T, FFN, device=dev, dtype=f32)
        self.do = torch.empty(T, D_MODEL, device=dev, dtype=f32)
        self.a16 = torch.empty(T, FFN, device=dev, dtype=torch.float16)
        self.scales = torch.empty(T, device=dev, dtype=f32)
        self.kc = torch.randn(TOKENS, NKV, HD, device=dev).half()
        self.vc = torch.randn(TOKENS, NKV, HD, device=dev).half()
        self.masks = []
        for u in range(TOKENS // UBATCH):
            n_kv = UBATCH * (u + 1)
            j = torch.arange(n_kv, device=dev)[None, :]
            t = torch.arange(T, device=dev)[:, None]
            m = torch.zeros(T, n_kv, device=dev)
            m[j > UBATCH * u + t] = float("-inf")
            self.masks.append(m.half())
        self.fa_ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        # K-split partials of the widest split among the layer's launches (summed in split order)
        launches = [[shapes["q"], shapes["k"], shapes["v"]], [shapes["o"]], [shapes["gate"], shapes["up"]],
                    [shapes["down"]]]
        need = 0
        for outs in launches:
            arr = (mx.GemmOut * len(outs))()
            for i, (N, K) in enumerate(outs):
                arr[i] = mx.GemmOut(None, N, 0, N, None, N)
            need = max(need, int(mx.lib().mi355x_gemm_workspace(self.wt, UBATCH, outs[0][1], arr, len(outs))))
        self.part = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        self._acc = {}
        self.timing = None

    # ---- op launchers (optionally bracketed by events on the launch stream) ----
    def _ev(self, kind, fn):
        if self.timing is None:
            fn()
            return
        torch = self.torch
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        self.timing.append((kind, s, e))

    def _pack(self, x, K, clear=None):
        """The activation pack; `clear` = the next GEMM's output when that GEMM adds a two-way K
        split into it (cleared by the pack in the same launch, as the backend does)."""
        mx = self.mx
        if clear is not None:
            self._ev("pack", lambda: mx.check(mx.lib().mi355x_pack_act_clear(
                int(self.wt == mx.F16_T), mx._ptr(x), x.stride(0), x.shape[0], K, mx._ptr(self.a16),
                mx._ptr(self.scales), mx._ptr(clear), clear.stride(0), clear.shape[1], mx.stream_handle()), "pack"))
            return
        fn = mx.lib().mi355x_pack_act_tiled if self.wt == mx.F16_T else mx.lib().mi355x_pack_act
        self._ev("pack", lambda: mx.check(fn(
            mx._ptr(x), x.stride(0), x.shape[0], K, mx._ptr(self.a16),
            mx._ptr(self.scales), mx.stream_handle()), "pack"))

    def _accumulates(self, K, outs):
        """Whether this launch adds a two-way K split into its (single) output."""
        mx = self.mx
        key = (K, tuple(N for _, N, _ in outs))
        if key not in self._acc:
            arr = (mx.GemmOut * len(outs))()
            for i, (_, N, _) in enumerate(outs):
                arr[i] = mx.GemmOut(None, N, 0, N, None, N)
            st = int(mx.lib().mi355x_gemm_accumulates(self.wt, UBATCH, K, arr, len(outs), self.part.numel()))
            if st < 0:
                raise RuntimeError(f"mi355x_gemm_accumulates: status {st}")
            self._acc[key] = st == 1 and len(outs) == 1
        return self._acc[key]

    def _gemm(self, K, outs, flops, zeroed=False):
        mx = self.mx
        arr = (mx.GemmOut * len(outs))()
        for i, (w, N, c) in enumerate(outs):
            arr[i] = mx.GemmOut(w.data_ptr(), N, 0, N, c.data_ptr(), c.stride(0))
        flags = 1 if zeroed else 0   # MI355X_GEMM_OUT_ZEROED
        self._ev("gemm", lambda: mx.check(mx.lib().mi355x_gemm_ws(
            self.wt, mx._ptr(self.a16), mx._ptr(self.scales), UBATCH, K, arr, len(outs),
            mx._ptr(self.part), self.part.numel(), flags, mx.stream_handle()), "gemm"))
        self.flops["gemm"] += flops

    def _mm(self, x, K, outs, flops):
        """pack + GEMM, the pack clearing the output when the GEMM accumulates into it."""
        acc = self._accumulates(K, outs)
        self._pack(x, K, clear=outs[0][2] if acc else None)
        self._gemm(K, outs, flops, zeroed=acc)

    def _fa(self, u, first=True):
        """The attention of micro-batch u; `first` for the micro-batch's first layer, which
        classifies the shared KQ mask's tiles into the workspace for the later layers."""
        n_kv = UBATCH * (u + 1)
        mx = self.mx
        q = self.qo.view(UBATCH, NH, HD).permute(1, 0, 2)
        k = self.kc[:n_kv].permute(1, 0, 2)
        v = self.vc[:n_kv].permute(1, 0, 2)
        m = self.masks[u]
        out = self.attn.view(UBATCH, NH, HD)
        self._ev("fa", lambda: mx.flash_attn(q, k, v, m, 1.0 / math.sqrt(HD), out=out, workspace=self.fa_ws,
                                             classes_ready=not first))
        self.flops["fa"] += 4.0 * NH * UBATCH * n_kv * HD

    def step(self):
        sh = self.shapes
        for u in range(TOKENS // UBATCH):
            for li, lw in enumerate(self.layers):
                M = UBATCH
                self._mm(self.x, D_MODEL, [(lw["q"], sh["q"][0], self.qo), (lw["k"], sh["k"][0], self.ko),
                                           (lw["v"], sh["v"][0], self.vo)],
                         2.0 * M * D_MODEL * (D_MODEL + 2 * NKV * HD))
                if UBATCH * (u + 1) >= self.fa_min_kv:
                    self._fa(u, first=li == 0)
                self._mm(self.attn, D_MODEL, [(lw["o"], D_MODEL, self.oo)], 2.0 * M * D_MODEL * D_MODEL)
                self._mm(self.x, D_MODEL, [(lw["gate"], FFN, self.go), (lw["up"], FFN, self.uo)],
                         2.0 * M * D_MODEL * 2 * FFN)
                self._mm(self.act, FFN, [(lw["down"], D_MODEL, self.do)], 2.0 * M * FFN * D_MODEL)

    def reset_counters(self, timing):
        self.flops = {"gemm": 0.0, "fa": 0.0}
        self.timing = [] if timing else None


def gemm_weight_bytes(route):
    per_w = 2.0 if route == "prepacked-q" else 144.0 / 256.0
    n = D_MODEL * D_MODEL * 2 + 2 * NKV * HD * D_MODEL + 3 * FFN * D_MODEL
    return n * per_w


def host_cpu():
    """CPU model, logical and physical core counts of this host, and the cores this process may
    run on (the box's share of the host)."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model == "unknown":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None and core is not None:
                    cores.add((phys, core))
                    phys = core = None
    except OSError:
        pass
    if phys is not None and core is not None:
        cores.add((phys, core))
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count() or 1
    return {"model": model, "logical_cores": os.cpu_count(), "physical_cores": len(cores) or None,
            "cores_allowed": allowed}


def cpu_baseline(prefill, threads):
    """The oracle (fp64 GEMM from the Q4_K payload, double attention; OpenMP) on a bounded sample
    of the same workload: layer 0, S tokens of the last micro-batch (n_kv 2048), all seven
    projections and the attention of those tokens. One warm-up pass, then at least 5 timed
    passes (until ~10 s, at most ~30 s); tokens/s = S / (median pass time * 32 layers)."""
    import numpy as np
    from oracle import oracle as O
    O.lib()
    cpu = host_cpu()
    env_threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    nt = threads or env_threads or cpu["cores_allowed"]
    S = 128
    X = O.fill_normal((S, D_MODEL), 5)
    Xf = O.fill_normal((S, FFN), 6)
    Qh = O.fill_normal((NH, S, HD), 7)
    K16 = O.f32_to_f16_bits(O.fill_normal((NKV, TOKENS, HD), 8))
    V16 = O.f32_to_f16_bits(O.fill_normal((NKV, TOKENS, HD), 9))
    t = np.arange(S)[:, None] + (TOKENS - S)
    M16 = O.f32_to_f16_bits(np.where(np.arange(TOKENS)[None, :] > t, -np.inf, 0.0).astype(np.float32))

    def one_pass():
        t0 = time.perf_counter()
        for name, (N, K) in prefill.shapes.items():
            O.mul_mat(O.Q4_K, prefill.host_q4[name], Xf if K == FFN else X, N, K, nthreads=nt)
        O.flash_attn(Qh, K16, V16, M16, 1.0 / math.sqrt(HD), nthreads=nt)
        return time.perf_counter() - t0

    one_pass()   # warm-up
    runs, t0 = [], time.perf_counter()
    while len(runs) < 5 or (time.perf_counter() - t0 < 10.0 and len(runs) < 64):
        runs.append(one_pass())
        if len(runs) >= 5 and time.perf_counter() - t0 > 30.0:
            break
    dt = float(np.median(runs))
    return {"value": round(S / (dt * L_LAYERS), 2), "unit": "tok/s", "cores": nt, "kind": "port",
            "cpu_model": cpu["model"], "logical_cores": cpu["logical_cores"],
            "physical_cores": cpu["physical_cores"], "cores_allowed": cpu["cores_allowed"],
            "threads": nt, "runs": len(runs), "median_pass_s": round(dt, 4),
            "sample": f"CPU oracle restatement (not ggml-cpu, which is absent here): layer 0 of the "
                      f"workload, {S} tokens of the last 512-token micro-batch (n_kv 2048): the 7 Q4_K "
                      f"projections as fp64 GEMM + double attention, OpenMP on {nt} threads; warm "
                      f"median of {len(runs)} passes, scaled x{L_LAYERS} layers"}


def time_ops(pf, reps=32):
    """Live HIP-event timing of each distinct launch of the step: `reps` launches of the same op
    are captured into a HIP graph, and events on the launch stream bracket replays of it, so the
    figure is GPU time per launch without host launch overhead (as in the replayed step). The
    GEMM launches cycle through the layers' weights, as the step does, so no launch finds its
    weight panel still cached by the one before."""
    torch = pf.torch
    sh = pf.shapes
    M = UBATCH
    L = len(pf.layers)
    lw = lambda i: pf.layers[i % L]
    ops = [
        ("pack", 0.0, 4 * L_LAYERS * 4, lambda i: pf._pack(pf.x, D_MODEL)),
        ("gemm", 2.0 * M * D_MODEL * (D_MODEL + 2 * NKV * HD), L_LAYERS * 4,
         lambda i: pf._gemm(D_MODEL, [(lw(i)["q"], sh["q"][0], pf.qo), (lw(i)["k"], sh["k"][0], pf.ko),
                                      (lw(i)["v"], sh["v"][0], pf.vo)], 0.0)),
        ("gemm", 2.0 * M * D_MODEL * D_MODEL, L_LAYERS * 4,
         lambda i: pf._gemm(D_MODEL, [(lw(i)["o"], D_MODEL, pf.oo)], 0.0)),
        ("gemm", 2.0 * M * D_MODEL * 2 * FFN, L_LAYERS * 4,
         lambda i: pf._gemm(D_MODEL, [(lw(i)["gate"], FFN, pf.go), (lw(i)["up"], FFN, pf.uo)], 0.0)),
        ("gemm", 2.0 * M * FFN * D_MODEL, L_LAYERS * 4,
         lambda i: pf._gemm(FFN, [(lw(i)["down"], D_MODEL, pf.do)], 0.0,
                            zeroed=pf._accumulates(FFN, [(None, D_MODEL, pf.do)]))),
    ]
    for u in range(TOKENS // UBATCH):
        kind = "fa" if UBATCH * (u + 1) >= pf.fa_min_kv else "fa-declined"
        ops.append((kind, 4.0 * NH * UBATCH * UBATCH * (u + 1) * HD, L_LAYERS, (lambda i, uu=u: pf._fa(uu, first=i == 0))))
    pf.reset_counters(False)
    out = []
    for kind, flops, per_step, fn in ops:
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn(0)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(reps):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(3):
            g.replay()
        e.record()
        torch.cuda.synchronize()
        out.append((kind, flops, per_step, s.elapsed_time(e) * 1e-3 / (3 * reps)))
    return out


def vendor_gemm(ops, reps=24):
    """The four projections at M = 512 through the vendor library, beside this backend's launch:
    torch.mm on fp16 operands with an fp32 output (hipBLASLt on ROCm; the same arithmetic: fp16
    products, fp32 accumulation, fp32 result), each weight cycled through enough copies to
    exceed the 256 MB last-level cache, timed with HIP events over `reps` back-to-back calls.
    The ours_us figures are time_ops' graph-replayed launches of the same shapes."""
    import torch
    names = ["qkv", "o", "gate_up", "down"]
    shapes = [(D_MODEL + 2 * NKV * HD, D_MODEL), (D_MODEL, D_MODEL), (2 * FFN, D_MODEL), (D_MODEL, FFN)]
    ours = [sec for kind, _, _, sec in ops if kind == "gemm"]
    out = {}
    for name, (N, K), mine in zip(names, shapes, ours):
        copies = max(2, int(600e6 // (N * K * 2)) + 1)
        g = torch.Generator(device="cuda")
        g.manual_seed(N + K)
        Ws = [torch.randn(N, K, device="cuda", dtype=torch.float16, generator=g) * 0.02 for _ in range(copies)]
        A = torch.randn(UBATCH, K, device="cuda", dtype=torch.float16, generator=g)
        try:
            mm = lambda i: torch.mm(A, Ws[i % copies].t(), out_dtype=torch.float32)
            mm(0)
            outdt = "f32"
        except (TypeError, RuntimeError):
            mm = lambda i: torch.mm(A, Ws[i % copies].t())
            outdt = "f16"
        for i in range(3):
            mm(i)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(reps):
            mm(i)
        e.record()
        torch.cuda.synchronize()
        us = s.elapsed_time(e) * 1e3 / reps
        flop = 2.0 * UBATCH * N * K
        out[name] = {"N": N, "K": K, "hipblaslt_us": round(us, 2), "hipblaslt_tflops": round(flop / us / 1e6, 1),
                     "ours_us": round(mine * 1e6, 2), "ours_tflops": round(flop / mine / 1e12, 1),
                     "speedup_vs_hipblaslt": round(us / (mine * 1e6), 3), "hipblaslt_out": outdt}
        del Ws, A
        torch.cuda.empty_cache()
    return out


def pmc_probe(pf):
    """One eager launch of each distinct op of the step (after one warm-up pass), then a plain
    device copy of 1 GiB, whose FETCH_SIZE / WRITE_SIZE read against its known 1 GiB in and out
    give the counters' scale. Prints the launch order so counter rows can be matched to ops."""
    torch = pf.torch
    lw, sh = pf.layers[0], pf.shapes
    pf.reset_counters(False)
    down_acc = pf._accumulates(FFN, [(None, D_MODEL, pf.do)])   # as in the step: the pack clears
    ops = [
        ("pack x[512,4096]", lambda: pf._pack(pf.x, D_MODEL)),
        ("gemm qkv 512x4096x6144", lambda: pf._gemm(D_MODEL, [(lw["q"], sh["q"][0], pf.qo),
                                                             (lw["k"], sh["k"][0], pf.ko),
                                                             (lw["v"], sh["v"][0], pf.vo)], 0.0)),
        ("gemm o 512x4096x4096", lambda: pf._gemm(D_MODEL, [(lw["o"], D_MODEL, pf.oo)], 0.0)),
        ("gemm gate/up 512x4096x28672", lambda: pf._gemm(D_MODEL, [(lw["gate"], FFN, pf.go),
                                                                  (lw["up"], FFN, pf.uo)], 0.0)),
        ("pack act[512,14336]", lambda: pf._pack(pf.act, FFN, clear=pf.do if down_acc else None)),
        ("gemm down 512x14336x4096", lambda: pf._gemm(FFN, [(lw["down"], D_MODEL, pf.do)], 0.0, zeroed=down_acc)),
        ("fa n_kv 2048", lambda: pf._fa(3)),
    ]
    for _, fn in ops:
        fn()
    torch.cuda.synchronize()
    for name, fn in ops:
        print(f"pmc-probe: {name}", flush=True)
        fn()
        torch.cuda.synchronize()
    src = torch.ones(1 << 28, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    print("pmc-probe: copy 1 GiB -> 1 GiB", flush=True)
    dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc-probe: done", flush=True)


def host_path(args):
    """The same prefill through the plugin boundary: every op of the step handed to
    mi355x_backend_graph_compute as host tensors, which uploads the inputs, runs the kernels
    and downloads dst before returning (the contract of the reference backend: no device-resident
    activations, no async slots). One graph_compute per group the ggml scheduler would form:
    {Q, K, V} (fused), {FLASH_ATTN_EXT, O}, {gate, up} (fused), {down}. Weights are per-layer Q4_K
    payloads in host memory with their own names, so the first pass builds the HBM weight cache
    (decoded, tiled fp16: the QUANT_RESIDENT route) and the second, timed, pass finds every
    weight resident. Prints one JSON line with the PCIe-inclusive rate.

    With --gguf PATH the model comes from a GGUF file instead (llama.cpp's tensor names, e.g. the
    random-init Llama-3-8B of llama3_gguf.py): its dims from the file's llama.* metadata, its
    weights passed to the backend as views of the memory-mapped file under their GGUF names, as a
    host's ggml hands a mapped model's tensors over."""
    import ctypes
    import numpy as np
    import ggml_mi355x as mx
    be = mx.Backend()
    be.set_quant_resident(1)
    T = UBATCH
    t0 = time.time()
    wg = mx.Graph()
    wts = []
    gguf = getattr(args, "gguf", None)
    if gguf:
        import gguf_io
        r = gguf_io.Reader(gguf)
        kv = r.kv
        if kv.get("general.architecture") != "llama":
            raise SystemExit(f"{gguf}: architecture {kv.get('general.architecture')!r}, not llama")
        d_model, ffn = int(kv["llama.embedding_length"]), int(kv["llama.feed_forward_length"])
        nh, nkv = int(kv["llama.attention.head_count"]), int(kv["llama.attention.head_count_kv"])
        hd = d_model // nh
        L = min(args.layers, int(kv["llama.block_count"]))
        gname = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
                 "up": "ffn_up", "down": "ffn_down"}
        shapes = {}
        for li in range(L):
            lw = {}
            for name, g in gname.items():
                tn = f"blk.{li}.{g}.weight"
                t, ne, _, _ = r.tensors[tn]
                shapes[name] = (int(ne[1]), int(ne[0]))
                lw[name] = wg._new(t, [int(ne[0]), int(ne[1])], name=tn, data=r.data(tn))
            wts.append(lw)
    else:
        d_model, ffn, nh, nkv, hd, L = D_MODEL, FFN, NH, NKV, HD, args.layers
        shapes = {"q": (d_model, d_model), "k": (nkv * hd, d_model), "v": (nkv * hd, d_model),
                  "o": (d_model, d_model), "gate": (ffn, d_model), "up": (ffn, d_model), "down": (d_model, ffn)}
        rng = np.random.default_rng(1234)
        base = {}
        for i, (name, (N, K)) in enumerate(shapes.items()):
            base[name] = synth_q4k(N, K, 0x5EED0000 + 80 + i)
        for li in range(L):
            lw = {}
            for name, (N, K) in shapes.items():
                q = base[name].copy()
                if li > 0:   # fresh nibbles under layer 0's block headers: valid Q4_K, distinct per layer
                    q.reshape(-1, 144)[:, 16:] = rng.integers(0, 256, (q.size // 144, 128), dtype=np.uint8)
                lw[name] = wg._new(mx.Q4_K, [K, N], name=f"blk.{li}.{name}.weight", data=q)
            wts.append(lw)
    rng = np.random.default_rng(1234)
    setup_s = time.time() - t0

    g = mx.Graph()
    f32 = lambda *n: np.zeros(int(np.prod(n)), dtype=np.float32)
    x = g._new(mx.F32, [d_model, T], data=rng.standard_normal(d_model * T).astype(np.float32))
    act = g._new(mx.F32, [ffn, T], data=rng.standard_normal(ffn * T).astype(np.float32))
    kc = g._new(mx.F16, [hd, nkv, TOKENS], data=rng.standard_normal(hd * nkv * TOKENS).astype(np.float16))
    vc = g._new(mx.F16, [hd, nkv, TOKENS], data=rng.standard_normal(hd * nkv * TOKENS).astype(np.float16))
    masks = []
    for u in range(TOKENS // T):
        n_kv = T * (u + 1)
        m = np.zeros((T, n_kv), dtype=np.float16)
        m[np.arange(n_kv)[None, :] > T * u + np.arange(T)[:, None]] = -np.inf
        masks.append(g._new(mx.F16, [n_kv, T], data=m.reshape(-1)))
    bufs = {n: f32(N, T) for n, (N, _) in shapes.items()}
    bufs["attn"] = f32(hd, nh, T)
    attn_cpu = g._new(mx.F32, [d_model, T], data=rng.standard_normal(d_model * T).astype(np.float32))

    def groups(li, u):
        """The graph_compute calls of layer li, micro-batch u."""
        n_kv = T * (u + 1)
        w = wts[li]
        mm = lambda name, src: g._new(mx.F32, [shapes[name][0], T], op=mx.OP_MUL_MAT, srcs=(w[name], src),
                                      data=bufs[name])
        q, k, v = mm("q", x), mm("k", x), mm("v", x)
        qv = g.permute_view(q, [hd, T, nh, 1], [4, d_model * 4, hd * 4, d_model * 4 * T])
        kv = g.permute_view(kc, [hd, n_kv, nkv, 1], [2, nkv * hd * 2, hd * 2, nkv * hd * 2 * n_kv])
        vv = g.permute_view(vc, [hd, n_kv, nkv, 1], [2, nkv * hd * 2, hd * 2, nkv * hd * 2 * n_kv])
        fa = g._new(mx.F32, [hd, nh, T], op=mx.OP_FLASH_ATTN_EXT, srcs=(qv, kv, vv, masks[u]), data=bufs["attn"])
        ctypes.memmove(ctypes.addressof(fa.op_params), (ctypes.c_float * 3)(1.0 / math.sqrt(hd), 0.0, 0.0), 12)
        fa2d = g.permute_view(fa, [d_model, T, 1, 1], [4, d_model * 4, d_model * 4 * T, d_model * 4 * T])
        # the attention is the backend's where it is claimed (n_kv >= FLASH_ATTN_MIN_KV); the
        # declined one is the host CPU's, and O then reads its result from host memory
        attn = [fa, fa2d, mm("o", fa2d)] if n_kv >= args.fa_min_kv else [mm("o", attn_cpu)]
        return [[q, k, v], attn, [mm("gate", x), mm("up", x)], [mm("down", act)]]

    calls = [grp for u in range(TOKENS // T) for li in range(L) for grp in groups(li, u)]

    def run():
        for nodes in calls:
            st = be.compute(nodes)
            if st != 0:
                raise RuntimeError(f"graph_compute status {st}")

    keys = ("bytes_up", "bytes_down", "pieces_up", "pieces_down", "up_copy_s", "up_wait_s", "down_copy_s",
            "down_wait_s", "copy_api_s", "weight_s")

    def run_split():
        """One more pass, each call's wall time and host-side copy accounting summed per group of
        the layer ({Q,K,V}, {attention, O}, {gate,up}, {down})."""
        per = [dict(calls=0, wall_s=0.0, **{k: 0.0 for k in keys}) for _ in range(4)]
        for i, nodes in enumerate(calls):
            h0 = be.host_stats()
            t0 = time.perf_counter()
            if be.compute(nodes) != 0:
                raise RuntimeError("graph_compute failed")
            dt = time.perf_counter() - t0
            h1 = be.host_stats()
            p = per[i % 4]
            p["calls"] += 1
            p["wall_s"] += dt
            for k in keys:
                p[k] += h1[k] - h0[k]
        return per

    t0 = time.time()
    run()                                       # builds the HBM weight cache
    first_s = time.time() - t0
    t0 = time.time()
    h0 = be.host_stats()
    run()
    sec = time.time() - t0
    h1 = be.host_stats()
    split = run_split()
    link = pinned_link_rate()
    names = ["qkv", "attn+o", "gate_up", "down"]
    per_call = {}
    for n, p in zip(names, split):
        c = max(p["calls"], 1)
        mb = (p["bytes_up"] + p["bytes_down"]) / c / 1e6
        per_call[n] = {"ms": round(p["wall_s"] / c * 1e3, 3), "MB_up": round(p["bytes_up"] / c / 1e6, 2),
                       "MB_down": round(p["bytes_down"] / c / 1e6, 2),
                       "link_floor_ms": round(mb / link["GBps_one_way"], 3) if link else None,
                       "pieces": round((p["pieces_up"] + p["pieces_down"]) / c, 1),
                       **{k.replace("_s", "_ms"): round(p[k] / c * 1e3, 3) for k in keys[4:]}}
    bytes_step = (h1["bytes_up"] - h0["bytes_up"]) + (h1["bytes_down"] - h0["bytes_down"])
    fb = be.cpu_fallbacks()
    routes = {r: be.route_ops(r) for r in ("prepacked-q", "fused-resident", "fa", "mt", "fused")}
    be.free()
    out = {"metric": "prefill tok/s through graph_compute (host buffers, PCIe-inclusive)",
           "value": round(TOKENS / sec, 1), "unit": "tok/s", "n_gpus": 1, "ms_per_prefill": round(sec * 1e3, 1),
           "higher_is_better": True, "dtype": "f16",
           "data": (f"weights memory-mapped from {os.path.basename(gguf)}, synthetic activations" if gguf
                    else "synthetic host tensors"),
           "config": {"workload": f"llama3-8b-shape Q4_K prefill, {TOKENS} tokens in {TOKENS // T} micro-batches "
                                  f"of {T}: {len(calls) // (TOKENS // T)} graph_compute calls per micro-batch",
                      "layers": L, "d_model": d_model, "ffn": ffn, "heads": nh, "kv_heads": nkv,
                      "route": "prepacked-q (QUANT_RESIDENT)"},
           "first_pass_s": round(first_s, 2), "host_setup_s": round(setup_s, 1), "cpu_fallbacks": fb,
           "GB_per_prefill": round(bytes_step / 1e9, 2), "pinned_link": link,
           "link_floor_tok_s": round(TOKENS / (bytes_step / (link["GBps_one_way"] * 1e9)), 1) if link else None,
           "fa_mirror_hits": h1["fa_mirror_hits"] - h0["fa_mirror_hits"],
           "per_call": per_call,
           "routes": routes,
           "scope": "the backend's ops only: FLASH_ATTN_EXT at n_kv < FLASH_ATTN_MIN_KV and every op "
                    "the backend does not claim run on the host CPU and are not timed"}
    return out


def pinned_link_rate(mb=256):
    """Pinned host <-> device copy rate on this box (torch: pinned host tensors, HIP events):
    each direction alone, then both at once. The floor of the host-buffer path is its bytes at
    the one-way rate (the box's link does not run both directions at full rate together)."""
    import torch
    if not torch.cuda.is_available():
        return None
    n = mb << 20
    h = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    h2 = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    d = torch.empty(n, dtype=torch.uint8, device="cuda")
    d2 = torch.empty(n, dtype=torch.uint8, device="cuda")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def timed(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    for _ in range(2):
        up = timed(lambda: d.copy_(h, non_blocking=True))
        down = timed(lambda: h.copy_(d, non_blocking=True))

    def both():
        with torch.cuda.stream(s1):
            d.copy_(h, non_blocking=True)
        with torch.cuda.stream(s2):
            h2.copy_(d2, non_blocking=True)
    both_s = timed(both)
    return {"GBps_up": round(n / up / 1e9, 1), "GBps_down": round(n / down / 1e9, 1),
            "GBps_one_way": round(2 * n / (up + down) / 1e9, 1), "GBps_both_at_once": round(2 * n / both_s / 1e9, 1),
            "MB": mb}


def graph_time_us(fn_of_i, n_calls, reps=3):
    """Mean device time of fn_of_i(i), i = 0 .. n_calls-1, captured once into a HIP graph and
    replayed `reps` times between HIP events on the launch stream."""
    import torch
    for i in range(min(n_calls, 3)):
        fn_of_i(i)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn_of_i(0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_calls):
            fn_of_i(i)
    g.replay()
    torch.cuda.synchronize()
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(reps):
        g.replay()
    s1.record()
    torch.cuda.synchronize()
    return s0.elapsed_time(s1) * 1e3 / (reps * n_calls)


def synth_blocks(wtype, N, K, seed):
    """Random but well-formed ggml blocks for a timing run: random codes under a fixed small
    fp16 scale (Q8_0: d | qs[32]; Q6_K: ql[128] qh[64] scales[16] | d; Q4_K from synth_q4k)."""
    import numpy as np
    if wtype == 12:
        return synth_q4k(N, K, seed)
    bs, bb = {8: (32, 34), 14: (256, 210), 39: (32, 17)}[wtype]
    blk = np.random.default_rng(seed).integers(0, 256, size=(N * K // bs, bb), dtype=np.uint8)
    d = np.array([0.0005], dtype=np.float16).view(np.uint8)
    if wtype == 8:
        blk[:, 0:2] = d
    elif wtype == 14:
        blk[:, 208:210] = d
    else:
        blk[:, 0] = 118   # MXFP4: the E8M0 block scale 2^-9, then 16 bytes of FP4 codes
    return blk.reshape(-1)


def mul_mat_one(spec):
    """One quantized MUL_MAT shape of the single-op sweep, alone: same weights, same rotation over
    weight copies, same entry point and workspace as configs_bench."""
    import numpy as np
    import torch
    import ggml_mi355x as mx
    tn, N, K, M = spec.split(",")
    N, K, M = int(N), int(K), int(M)
    wt = {"Q8_0": mx.Q8_0, "Q4_K": mx.Q4_K, "Q6_K": mx.Q6_K, "Q4_0": mx.Q4_0, "Q5_K": mx.Q5_K, "MXFP4": mx.MXFP4}[tn]
    P = synth_blocks(wt, N, K, 0x5EED0000 + 64)
    w0 = mx.upload_weight(wt, P, N, K)
    ncopy = max(3, min(64, math.ceil(320e6 / w0.numel())))
    ws = [w0] + [w0.clone() for _ in range(ncopy - 1)]
    x = torch.randn(M, K, device="cuda")
    out = torch.empty(M, N, device="cuda")
    wsp = torch.empty(max(1, int(mx.lib().mi355x_mul_mat_workspace_for(wt, N, K, M))), dtype=torch.uint8, device="cuda")
    us = graph_time_us(lambda i: mx.mul_mat(wt, ws[i % ncopy], N, K, x, out, wsp), max(ncopy, 64))
    nbytes = P.nbytes + M * K * 4 + M * N * 4
    return {"case": f"MUL_MAT {tn} N={N} K={K} M={M}", "us": round(us, 2), "tflops": round(2.0 * M * N * K / us / 1e6, 1),
            "GBps": round(nbytes / us / 1e3, 1), "decode_first": int(mx.lib().mi355x_mul_mat_decode_first(wt, M, N, K))}


def configs_bench(args, subset=False, print_line=True):
    """The single-op configurations, each through the C ABI entry the backend uses for it and
    against the roofline that bounds it (arithmetic intensity against the 2.5 PFLOP/s / 8 TB/s
    ridge of ~312 FLOP/byte). MUL_MAT: mi355x_mul_mat (activation pack + GEMM) on an HBM-resident
    weight (F16 in the tiled fp16 layout; quantized types as ggml blocks, decoded in the GEMM),
    bytes = weight at its stored size + F32 activations + F32 output; the weight rotates over
    enough copies (>= 320 MB) that no call finds it in the 256 MB last-level cache.
    FLASH_ATTN_EXT: mi355x_flash_attn, causal mask, FLOP = the dense rectangle 4 H T n_kv d (the
    causal-visible share is reported beside it)."""
    import numpy as np
    import torch
    import ggml_mi355x as mx
    cases = {}

    def record(name, us, flop, nbytes, extra=None):
        ai = flop / nbytes
        tf, gbs = flop / us / 1e6, nbytes / us / 1e3
        bound = "mfma" if ai >= PEAK_F16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9) else "hbm"
        frac = tf / PEAK_F16_TFLOPS if bound == "mfma" else gbs / PEAK_HBM_GBS
        cases[name] = {"us": round(us, 2), "tflops": round(tf, 1), "GBps": round(gbs, 1),
                       "ai": round(ai, 1), "bound": bound, "frac": round(frac, 4), **(extra or {})}
        print(f"{name}: {us:8.2f} us  {tf:7.1f} TFLOP/s  {gbs:7.1f} GB/s  ({bound}, frac {frac:.3f})",
              file=sys.stderr, flush=True)

    def mul_mat_case(name, wtype, dev_type, payload, N, K, Ms):
        w0 = mx.upload_weight(wtype, payload, N, K)
        if dev_type == mx.F16_T:
            w0 = mx.tile_f16(wtype, w0, N, K)
        ncopy = max(3, min(64, math.ceil(320e6 / w0.numel())))
        ws = [w0] + [w0.clone() for _ in range(ncopy - 1)]
        for M in Ms:
            x = torch.randn(M, K, device="cuda")
            out = torch.empty(M, N, device="cuda")
            wsp = torch.empty(max(1, int(mx.lib().mi355x_mul_mat_workspace_for(dev_type, N, K, M))),
                              dtype=torch.uint8, device="cuda")
            us = graph_time_us(lambda i: mx.mul_mat(dev_type, ws[i % ncopy], N, K, x, out, wsp), ncopy)
            record(f"{name} M={M}", us, 2.0 * M * N * K, payload.nbytes + M * K * 4 + M * N * 4)
        del ws
        torch.cuda.empty_cache()

    # F16 weight [8192, 2048], activations [512, 2048]
    W = (np.random.default_rng(0x5EED0000 + 16).standard_normal((8192, 2048), dtype=np.float32) * 0.02)
    mul_mat_case("MUL_MAT F16 N=8192 K=2048", mx.F16, mx.F16_T, W.astype(np.float16).view(np.uint16),
                 8192, 2048, [512])
    # quantized sweep, the weight decoded per call (inside the GEMM, or first into tiled fp16 where
    # mi355x_mul_mat_decode_first says so); the default bench line carries one shape of it for
    # each type (K 3072, N 8192)
    for ti, (wt, tn) in enumerate(((mx.Q8_0, "Q8_0"), (mx.Q4_K, "Q4_K"), (mx.Q6_K, "Q6_K"))):
        for si, (K, N) in enumerate(((3072, 3072), (3072, 8192), (8192, 3072))):
            if subset and (K, N) != (3072, 8192):
                continue
            P = synth_blocks(wt, N, K, 0x5EED0000 + 32 + 4 * ti + si)
            mul_mat_case(f"MUL_MAT {tn} N={N} K={K}", wt, wt, P, N, K, [32, 128, 512, 2048])
    # FLASH_ATTN_EXT prefill: 32 query / 8 KV heads, d 128, 512 queries, causal
    T, H, HK, D = 512, 32, 8, 128
    for n_kv in (1024, 4096, 8192):
        q = torch.randn(T, H, D, device="cuda")
        kc = torch.randn(n_kv, HK, D, device="cuda").half()
        vc = torch.randn(n_kv, HK, D, device="cuda").half()
        j = torch.arange(n_kv, device="cuda")[None, :]
        t = torch.arange(T, device="cuda")[:, None]
        m = torch.where(j > n_kv - T + t, float("-inf"), 0.0).half()
        out = torch.empty(T, H, D, device="cuda")
        wsp = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        us = graph_time_us(lambda i: mx.flash_attn(q.permute(1, 0, 2), kc.permute(1, 0, 2), vc.permute(1, 0, 2),
                                                   m, 1.0 / math.sqrt(D), out=out, workspace=wsp), 8)
        visible = 4.0 * H * D * sum(n_kv - T + tt + 1 for tt in range(T))
        record(f"FLASH_ATTN_EXT n_kv={n_kv}", us, 4.0 * H * T * n_kv * D,
               T * H * D * 4 + 2 * HK * n_kv * D * 2 + T * n_kv * 2 + T * H * D * 4,
               {"tflops_causal_visible": round(visible / us / 1e6, 1)})
        del q, kc, vc, m, out, wsp
    torch.cuda.empty_cache()
    # FLASH_ATTN_EXT with the absorbed MLA's head dims (DeepSeek-style: keys of 576, values the
    # first 512 of them), 16 query heads on one KV head, 512 queries over 4096 keys, causal: the
    # two-GEMM path for head dims past 256
    T, H, HK, D, DV, n_kv = 512, 16, 1, 576, 512, 4096
    q = torch.randn(T, H, D, device="cuda")
    kc = torch.randn(n_kv, HK, D, device="cuda").half()
    j = torch.arange(n_kv, device="cuda")[None, :]
    t = torch.arange(T, device="cuda")[:, None]
    m = torch.where(j > n_kv - T + t, float("-inf"), 0.0).half()
    out = torch.empty(T, H, DV, device="cuda")
    kview = kc.permute(1, 0, 2)
    wsp = torch.empty(mx.flash_attn_workspace(q.permute(1, 0, 2), kview, kview[:, :, :DV], m, out) + 256,
                      dtype=torch.uint8, device="cuda")
    us = graph_time_us(lambda i: mx.flash_attn(q.permute(1, 0, 2), kview, kview[:, :, :DV], m, 1.0 / math.sqrt(D),
                                               out=out, workspace=wsp), 8)
    visible = 2.0 * H * (D + DV) * sum(n_kv - T + tt + 1 for tt in range(T))
    record(f"FLASH_ATTN_EXT absorbed MLA 576/512 n_kv={n_kv}", us, 2.0 * H * T * n_kv * (D + DV),
           T * H * D * 4 + HK * n_kv * D * 2 + T * n_kv * 2 + T * H * DV * 4,
           {"tflops_causal_visible": round(visible / us / 1e6, 1)})
    del q, kc, m, out, wsp
    torch.cuda.empty_cache()
    if subset or not print_line:
        return cases
    print(json.dumps({
        "metric": "single-op configurations vs their rooflines (MI355X peaks: 2.5 PFLOP/s fp16, 8 TB/s)",
        "n_gpus": 1, "dtype": "f16", "data": "synthetic (N(0,0.02) / random-code weights, N(0,1) activations)",
        "cases": cases}))


def moe_bench(args):
    """MUL_MAT_ID expert GEMM at the mixture-of-experts prefill shape: 128 experts, top-8 routing
    from a softmax over N(0, 1) router logits (ties to the lower index), 512 tokens, d_model 2048,
    expert FFN 768; gate/up [128 x 768 x 2048] (b: one row per token) and down [128 x 2048 x 768]
    (b: one row per token and slot), Q4_K experts quantized from N(0, 0.02), F32 activations.
    Each op is timed through mi355x_mul_mat_id (pack, bucketing and grouped GEMM) on three
    copies of its expert stack, cycled so no launch finds its weights in the 256 MB last-level
    cache, 8 calls per captured HIP graph, HIP events around the replays on the launch stream.
    The bound is HBM: bytes = expert weights at their stored size + F32 activations in + F32
    outputs, each counted once."""
    import numpy as np
    import torch
    import ggml_mi355x as mx
    E, U, T, DM, FF = 128, 8, 512, 2048, 768
    logits = np.random.default_rng(0x5EED0000 + 64).standard_normal((T, E), dtype=np.float32)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :U].astype(np.int32)   # softmax is monotone
    idt = torch.from_numpy(ids).cuda()
    # each stack in the layout the backend caches it in: regrouped by 32 rows
    main = moe_stack(args, mx.Q4_K_X, lambda n, k, seed: synth_q4k(n, k, seed), E, U, T, DM, FF, idt)
    others = {}
    if not getattr(args, "quick", False):
        for tn, lay, wt in (("Q8_0", mx.Q8_0_X, mx.Q8_0), ("Q6_K", mx.Q6_K_X, mx.Q6_K), ("MXFP4", mx.MXFP4_X, mx.MXFP4)):
            others[tn] = moe_stack(args, lay, lambda n, k, seed, wt=wt: synth_blocks(wt, n, k, seed),
                                   E, U, T, DM, FF, idt)
    gbs = main["GBps"]
    return {
        "metric": "MUL_MAT_ID expert GEMM GB/s (128 experts, top-8, 512 tok, d 2048, FFN 768, Q4_K)",
        "value": gbs, "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "f16", "data": "synthetic (Q4_K experts from N(0,0.02), random-code Q8_0 / Q6_K / MXFP4 "
                                "experts, N(0,1) activations and router logits)",
        "config": {"workload": "MoE prefill expert GEMMs: gate/up and down, cold expert stacks",
                   "experts": E, "top_k": U, "tokens": T, "d_model": DM, "ffn": FF},
        "ops": main["ops"],
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None},
        "other_stacks": others,
    }


def moe_stack(args, wt, synth, E, U, T, DM, FF, idt):
    """Times gate/up and down of one expert-stack weight type (see moe_bench)."""
    import torch
    import ggml_mi355x as mx
    ops = {}
    tot_us = tot_bytes = 0.0
    for i, (name, N, K, ne11) in enumerate((("gate/up", FF, DM, 1), ("down", DM, FF, U))):
        P = synth(E * N, K, 0x5EED0000 + 65 + i)
        copies = [mx.upload_weight(wt, P, E * N, K) for _ in range(3)]
        X = torch.randn(T, ne11, K, device="cuda")
        out = torch.empty(T, U, N, device="cuda")
        ws = torch.empty(1 << 26, dtype=torch.uint8, device="cuda")
        cyc = [0]

        def run():
            w = copies[cyc[0] % 3]
            cyc[0] += 1
            mx.mul_mat_id(wt, w, E, N, K, X, idt, out=out, workspace=ws)
        for _ in range(3):
            run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for _ in range(8):
                run()
        g.replay()
        torch.cuda.synchronize()
        reps = max(2, args.steps // 2)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(reps):
            g.replay()
        s1.record()
        torch.cuda.synchronize()
        us = s0.elapsed_time(s1) * 1e3 / (8 * reps)
        nbytes = P.nbytes + X.numel() * 4 + out.numel() * 4
        flop = 2.0 * T * U * N * K
        ops[name] = {"us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1), "tflops": round(flop / us / 1e6, 1),
                     "weight_MB": round(P.nbytes / 1e6, 1)}
        tot_us += us
        tot_bytes += nbytes
        del copies, X, out, ws, g
        torch.cuda.empty_cache()
    gbs = tot_bytes / tot_us / 1e3
    return {"GBps": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4), "ops": ops}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              f"the multi-GPU sharding is a design note, not a benchmark.", file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    if args.mul_mat:
        print(json.dumps(mul_mat_one(args.mul_mat)), flush=True)
        return
    if args.pmc_probe:
        pmc_probe(Prefill(args.route, 1))
        return
    if args.moe:
        print(json.dumps(moe_bench(args)), flush=True)
        return
    if args.configs:
        configs_bench(args)
        return
    if args.host_path:
        print(json.dumps(host_path(args)), flush=True)
        return
    pf = Prefill(args.route, args.layers, args.fa_min_kv)

    pf.reset_counters(False)
    for _ in range(args.warmup):
        pf.step()
    torch.cuda.synchronize()

    # the step is captured once into a HIP graph and replayed: ~1300 launches per step would
    # otherwise be bound by host launch overhead, not by the GPU
    graph = None
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            pf.step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            pf.step()
        graph.replay()
        torch.cuda.synchronize()
    except Exception as exc:  # eager steps still measure the same work
        print(f"bench.py: graph capture unavailable ({exc}); timing eager steps", file=sys.stderr)
        graph = None

    steps = args.steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        if graph is not None:
            graph.replay()
        else:
            pf.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = wall / steps * 1e3
    scale_layers = L_LAYERS / args.layers
    tok_s = TOKENS / (wall / steps) / scale_layers

    ops = time_ops(pf)
    per = {}
    for kind, flops, per_step, sec in ops:
        d = per.setdefault(kind, {"flops": 0.0, "sec": 0.0, "launches": 0})
        d["flops"] += flops * per_step
        d["sec"] += sec * per_step
        d["launches"] += per_step
    gemm, fa = per["gemm"], per["fa"]
    declined = per.get("fa-declined")
    traffic, traffic_src = gemm_traffic(args.route)
    # causal-visible share of the claimed attention (keys a query may see), besides the rectangle
    fa_visible = sum(4.0 * NH * HD * sum(UBATCH * u + t + 1 for t in range(UBATCH)) * L_LAYERS
                     for u in range(TOKENS // UBATCH) if UBATCH * (u + 1) >= args.fa_min_kv)
    gemm_tf = gemm["flops"] / gemm["sec"] / 1e12
    fa_tf = fa["flops"] / fa["sec"] / 1e12
    wbytes = gemm_weight_bytes(args.route) * L_LAYERS * (TOKENS // UBATCH)
    kern_ms = sum(d["sec"] for d in per.values()) * 1e3
    res = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (random-init Q4_K weights from N(0,0.02), N(0,1) activations and KV)",
        "config": {"workload": "llama3-8b-shape Q4_K prefill, 2048 tokens in 4 micro-batches of 512: "
                               "the backend-claimed ops (fused QKV, FLASH_ATTN_EXT at n_kv >= "
                               f"{args.fa_min_kv}, O, fused gate/up, down) x 32 layers, inputs resident "
                               "in HBM; not an end-to-end prefill (see host_path)",
                   "layers": args.layers, "route": args.route, "global_batch": TOKENS,
                   "ubatch": UBATCH, "parallelism": "none (1 GPU)",
                   "replay": "hip graph" if graph is not None else "eager"},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tf, 1), "peak": PEAK_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gemm_tf / PEAK_F16_TFLOPS, 4),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": ("gemm_f16_kernel / gemm_f16_cols_kernel (LDS-DMA, fp16 MFMA 32x32x16)" if args.route == "prepacked-q"
                                else "gemm_kernel<Q4_K> (register-staged, Q4_K decoded into LDS, fp16 MFMA 32x32x16)"),
                     "avg_launch_us": round(gemm["sec"] / gemm["launches"] * 1e6, 2),
                     "flop_per_launch": round(gemm["flops"] / gemm["launches"])},
        "kernels": {
            "gemm": {"tflops": round(gemm_tf, 1), "frac_peak": round(gemm_tf / PEAK_F16_TFLOPS, 4),
                     "ms_per_step": round(gemm["sec"] * 1e3, 3), "launches_per_step": gemm["launches"],
                     "weight_GBps": round(wbytes / gemm["sec"] / 1e9, 1)},
            "flash_attn": {"tflops": round(fa_tf, 1), "frac_peak": round(fa_tf / PEAK_F16_TFLOPS, 4),
                           "ms_per_step": round(fa["sec"] * 1e3, 3), "launches_per_step": fa["launches"],
                           "flop_count": "dense rectangle 4*H*T*n_kv*d",
                           "tflops_causal_visible": round(fa_visible / fa["sec"] / 1e12, 1),
                           "declined_n_kv_512_us": (round(declined["sec"] / declined["launches"] * 1e6, 2)
                                                    if declined else None)},
            "pack_act": {"ms_per_step": round(per["pack"]["sec"] * 1e3, 3)},
            "kernel_sum_ms_per_step": round(kern_ms, 3),
            "per_op_us": {f"{k}:{i}": round(sec * 1e6, 2) for i, (k, _, _, sec) in enumerate(ops)},
        },
        "setup_s": round(pf.setup_s, 1),
    }
    if not args.quick:
        res["kernels"]["gemm_vs_hipblaslt"] = vendor_gemm(ops)
    if not (args.no_cpu_baseline or args.quick):
        res["cpu_baseline"] = cpu_baseline(pf, args.cpu_threads)
    if not args.quick:
        # the single-op configurations and the plugin-boundary rate, as further keys of the line
        host_q4 = pf.host_q4
        del pf
        torch.cuda.empty_cache()
        t0 = time.time()
        res["configs"] = configs_bench(args, print_line=False)
        moe = moe_bench(args)
        res["configs"]["MUL_MAT_ID 128e top-8 Q4_K"] = {
            "GBps": moe["value"], "frac": moe["roofline"]["frac"], "bound": "hbm", "ops": moe["ops"]}
        for tn, st in moe["other_stacks"].items():
            res["configs"][f"MUL_MAT_ID 128e top-8 {tn}"] = {"bound": "hbm", **st}
        res["configs_s"] = round(time.time() - t0, 1)
        t0 = time.time()
        res["host_path"] = host_path(args)
        res["host_path"]["wall_s"] = round(time.time() - t0, 1)
        del host_q4
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
