"""Benchmark of the MI355X decode hot path (one GPU).

Default workload: one FP8 MoE FFN decode step at batch 1 -- router top-8 over 128
experts from fresh N(0, 1) logits, fused gate/up + SiLU*mul, down projection and
slot-order weighted combine, hidden 4096, expert intermediate 1536, e4m3 weights with
128x128-block fp32 scales quantised from N(0, 0.02) -- run through
oom_moe_decode_fp8 with inputs resident in HBM. Two full sets of 128 experts
(2 x 2.42 GB) alternate between steps so weights stream from HBM, not from the
256 MB Infinity Cache.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--rounds R]
                    [--config decode1|decode16|layer1|layer16|nvfp4|offload|attn|turbo|prefill|nvfp4-prefill|gemv|copy|bf16]

After W untimed warm-up steps, R rounds (default 5) of K back-to-back steps are timed with
HIP events on the launch stream; `value` is the median round, and `timing` holds every
round's figure and their spread. Prints one JSON line (rank 0): metric, value (us/token), roofline of the step's
kernels against 8 TB/s HBM, and the reference CPU path (oracle restatement) timed on
this host's cores over a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
METRIC = "MoE FP8 decode layer µs/token + achieved HBM GB/s (% of MI355X peak), 1 GPU"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_rounds(step, first, args, stream, torch, per_step=1):
    """Median milliseconds per step over args.rounds rounds of args.steps back-to-back
    calls step(first + r * args.steps + i): each round between two events on `stream` (the
    launch stream), the device synchronised before and after. Returns (median, timing
    record: rounds, per-round ms per step, spread = (max - min) / median). per_step divides
    each round's figure further (calls a step makes)."""
    per = []
    for r in range(args.rounds):
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(args.steps):
            step(first + r * args.steps + i)
        b.record(stream)
        torch.cuda.synchronize()
        per.append(a.elapsed_time(b) / (args.steps * per_step))
    med = sorted(per)[len(per) // 2] if len(per) % 2 else sum(sorted(per)[len(per) // 2 - 1:len(per) // 2 + 1]) / 2
    return med, {"rounds": len(per), "steps_per_round": args.steps, "round_ms": [round(v, 6) for v in per],
                 "spread": (max(per) - min(per)) / med}


def quantize_blocks_dev(w, torch):
    """e4m3 codes and 128x128 fp32 scales of a bf16-valued [n, k] tensor on the device:
    scale = block absmax / 448 (1 for a zero block), q = e4m3(w / scale) rounded to
    nearest even and saturated at +-448 (crates/oominf-core/src/fp8.rs:52-88 per block)."""
    n, k = w.shape
    b = w.reshape(n // 128, 128, k // 128, 128)
    amax = b.abs().amax(dim=(1, 3))
    s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (b / s[:, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).reshape(n, k)
    return q, s.contiguous()


def make_expert_set(E, geo, stride, seed, torch):
    """[E, stride] uint8 records of E experts, weights N(0, 0.02) rounded to bf16, built
    a few experts at a time on the device."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    buf = torch.zeros((E, stride), dtype=torch.uint8, device="cuda")
    H, I = geo.hidden, geo.inter
    parts = [(geo.gate_weight, geo.gate_scale, I, H), (geo.up_weight, geo.up_scale, I, H),
             (geo.down_weight, geo.down_scale, H, I)]
    chunk = 16
    for e0 in range(0, E, chunk):
        ne = min(chunk, E - e0)
        for wo, so, n, k in parts:
            w = (torch.randn((ne * n, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16).float()
            q, s = quantize_blocks_dev(w, torch)
            buf[e0:e0 + ne, wo:wo + n * k] = q.reshape(ne, n * k)
            buf[e0:e0 + ne, so:so + (n // 128) * (k // 128) * 4] = s.reshape(ne, -1).contiguous().view(torch.uint8)
    return buf


def copy_bandwidth(torch, nbytes=1 << 30, reps=10):
    """GB/s of a plain device copy of `nbytes` (read + write counted), the STREAM-like
    figure quoted beside the 8 TB/s peak; also the calibration kernel of the PMC runs."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.mul(src, 1.0, out=dst)  # one elementwise kernel: reads and writes nbytes
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        torch.mul(src, 1.0, out=dst)
    b.record()
    torch.cuda.synchronize()
    return 2 * nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9


def measured_traffic(config):
    """HBM bytes per launch of the step's kernel from the committed rocprofv3 PMC
    summary (profiles/traffic.json: FETCH_SIZE and WRITE_SIZE per dispatch, each
    scaled by what the counter reads for a copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)[config]
        return float(t["bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def zipf_bias(E, s, seed):
    """Per-expert router-logit bias of a Zipf(s) popularity prior: the expert of
    popularity rank r (a seeded permutation) gets ln p_r = -s ln(r + 1) + const."""
    import numpy as np

    perm = np.random.default_rng(seed).permutation(E)
    bias = np.empty(E, dtype=np.float32)
    bias[perm] = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    return bias


def usable_cores() -> int:
    """Every core this process may run on: the affinity mask, within the job's CPU share
    when the environment states one (OMP_NUM_THREADS, as the batch system sets it)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, n)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_decode(host_recs, geo, E, k, T, zipf, budget_s=10.0):
    """The reference CPU path (oracle restatement of crates/oominf-cpu) on this host:
    router -> plan -> HostExperts -> slot-order combine per step, fresh logits each
    step, for about `budget_s` seconds. Returns (us_per_token, cores, steps)."""
    import numpy as np

    import oracle

    cores = usable_cores()
    rng = np.random.default_rng(5)
    x = oracle.bf16_to_f32(oracle.bf16_from_f32(rng.standard_normal((T, geo.hidden)).astype(np.float32)))
    t0 = time.perf_counter()
    steps = 0
    while True:
        logits = rng.standard_normal((T, E)).astype(np.float32)
        if zipf is not None:
            logits += zipf_bias(E, zipf, 7)
        ids, w = oracle.router_topk(logits, k)
        experts, off, tok, slot = oracle.moe_plan(ids, E)
        jobs = [tok[off[i]:off[i + 1]] for i in range(len(experts))]
        y = oracle.host_experts(geo, [host_recs[e] for e in experts], jobs, x, cores)
        oracle.moe_combine_slots(y, slot, w)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s and steps >= 3:
            break
    return el / steps / T * 1e6, cores, steps


def bench_decode(args, T, zipf, config):
    import numpy as np
    import torch

    import homelab_amd as hip

    E, k, H, I = 128, 8, 4096, 1536
    geo = hip.record_geometry(H, I)
    stride = hip.record_stride(geo)
    log(f"bench: decode T={T} E={E} k={k} H={H} I={I}; building 2 expert sets of {E * stride / 1e9:.2f} GB")
    sets = [make_expert_set(E, geo, stride, 1234 + s, torch) for s in range(2)]
    addrs = [torch.tensor([b.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
             for b in sets]
    n = args.warmup + args.rounds * args.steps
    g = torch.Generator(device="cuda")
    g.manual_seed(99)
    logits = torch.randn((n, T, E), generator=g, device="cuda")
    if zipf is not None:
        logits = logits + torch.from_numpy(zipf_bias(E, zipf, 7)).cuda()
    logits = logits.contiguous()
    x = (torch.randn((T, H), generator=g, device="cuda")).to(torch.bfloat16)
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ids = torch.empty((n, T, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((n, T, k), dtype=torch.float32, device="cuda")
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(T, E, k, geo), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def step(i):
        hip.moe_decode_fp8(logits[i], x, addrs[i % 2], k, geo, ids[i], wts[i], out, ws, stream)

    for i in range(args.warmup):
        step(i)
    ms, timing = time_rounds(step, args.warmup, args, stream, torch)
    # algorithmic bytes: each distinct routed expert's weights and scales once, x and out
    idn = ids[args.warmup:].cpu().numpy()
    distinct = np.array([len(np.unique(s)) for s in idn])
    per_expert = 3 * H * I + 3 * ((H + 127) // 128) * ((I + 127) // 128) * 4
    bytes_step = float(distinct.mean()) * per_expert + 2 * T * H * 2
    gbs = bytes_step / (ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": ms * 1e3 / T,
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "timing": timing,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 weights, bf16 activations, fp32 accumulate",
        "data": "synthetic",
        "config": {"workload": f"MoE FFN decode step, batch {T}: 128 experts top-8, hidden 4096, inter 1536, "
                               "e4m3 128x128-block-scaled weights from N(0,0.02), bf16 x, fresh N(0,1) logits"
                               + (f" + Zipf({zipf}) bias" if zipf else "") + "; 2 expert sets alternate past the MALL",
                   "batch": T, "experts": E, "top_k": k, "hidden": H, "inter": I,
                   "distinct_experts_per_step": float(distinct.mean())},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": measured_traffic(config),
                     "kernel": ("moe_decode_fused_kernel" if T == 1 else "moe_batch_kernel") + " (oom_moe_decode_fp8)",
                     "algorithmic_bytes_per_step": bytes_step, "copy_gbs": copy_bandwidth(torch)},
    }
    if not args.no_cpu:
        host = sets[0].cpu().numpy()
        import oracle

        ogeo = oracle.record_geometry(H, I)
        us, cores, nsteps = cpu_baseline_decode([host[e] for e in range(E)], ogeo, E, k, T, zipf, args.cpu_seconds)
        res["cpu_baseline"] = {"value": us, "unit": "us/token", "cores": cores, "kind": "port",
                               "sample": f"{nsteps} steps of the same batch-{T} decode MoE layer (fresh logits), "
                                         f"oracle restatement of crates/oominf-cpu HostExperts on {cpu_model()}"}
    return res


def cpu_baseline_gemv(x, q, scale, budget_s):
    """The oracle's restatement of the reference FP8 GEMV (crates/oominf-cuda/kernels/ops.cu:339-440
    arithmetic) on this host's cores, the rows split evenly over one thread each, for
    about `budget_s` seconds. Returns (us_per_call, threads, calls)."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle

    N = q.shape[0]
    threads = usable_cores()
    bounds = np.linspace(0, N, threads + 1).astype(int)
    parts = [(np.ascontiguousarray(q[a:b]), np.ascontiguousarray(scale[a:b])) for a, b in zip(bounds[:-1], bounds[1:])]

    def one(i):
        qq, ss = parts[i]
        return oracle.gemv_fp8(x, qq, ss, oracle.SCALE_ROW)

    t0 = time.perf_counter()
    calls = 0
    with ThreadPoolExecutor(threads) as pool:
        while True:
            list(pool.map(one, range(threads)))
            calls += 1
            el = time.perf_counter() - t0
            if el >= budget_s and calls >= 3:
                break
    return el / calls * 1e6, threads, calls


def bench_gemv(args):
    """One FP8 weight-only GEMV, batch 1: y = W x with W 4096 x 4096 e4m3 quantised from
    N(0, 0.02) with per-output-row absmax fp32 scales, x 1 x 4096 bf16 N(0, 1), fp32
    accumulate, bf16 y (oom_gemv_fp8, OOM_SCALE_ROW). 48 weight copies (805 MB) rotate
    between calls so W streams from HBM, not from the 256 MB MALL. A step is one pass over
    the 48 copies (48 calls): a ~5 us call timed 100 at a time is dominated by the first
    launch after the synchronisation; `value` is per call."""
    import numpy as np
    import torch

    import homelab_amd as hip

    N = K = 4096
    copies = 48
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    qs = torch.empty((copies, N, K), dtype=torch.uint8, device="cuda")
    ss = torch.empty((copies, N), dtype=torch.float32, device="cuda")
    for c in range(copies):
        w = torch.randn((N, K), generator=g, device="cuda") * 0.02
        amax = w.abs().amax(dim=1)
        sc = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
        qs[c] = (w / sc[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
        ss[c] = sc
    x = torch.randn((1, K), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
    ws_bytes = hip.gemv_fp8_workspace_size(1, N, K)
    ws = torch.zeros(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    # each copy's C-ABI arguments built once: the timed loop is one C call per GEMV (the
    # Python wrapper's tensor indexing and checks cost more host time than the kernel)
    fn = hip.lib().oom_gemv_fp8
    cargs = [(hip._ptr(x), hip._dtype_code(x), hip._ptr(qs[c]), hip._ptr(ss[c]), hip.SCALE_ROW, hip._ptr(y),
              hip._dtype_code(y), 1, N, K, hip._ptr(ws), ws_bytes, hip._stream(stream)) for c in range(copies)]
    hip.gemv_fp8(x, qs[0], ss[0], hip.SCALE_ROW, y, ws, stream)  # the wrapper's own checks, once

    def step(i):
        for c in range(copies):
            rc = fn(*cargs[c])
            if rc:
                hip.check(rc)

    for i in range(args.warmup):
        step(i)
    ms, timing = time_rounds(step, 0, args, stream, torch, per_step=copies)  # per call
    bytes_call = N * K + N * 4 + K * 2 + N * 2
    gbs = bytes_call / (ms * 1e-3) / 1e9
    res = {
        "metric": "FP8 weight-only GEMV us/call + achieved HBM GB/s (% of MI355X peak), 1 GPU",
        "value": ms * 1e3, "unit": "us/call", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms * copies, "calls_per_step": copies, "timing": timing, "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8-e4m3 weights, bf16 x and y, fp32 accumulate", "data": "synthetic",
        "config": {"workload": "FP8 GEMV, batch 1: W 4096x4096 e4m3 from N(0,0.02) with per-row absmax fp32 scales, "
                               "x 1x4096 bf16 N(0,1), bf16 y; 48 weight copies rotate past the MALL",
                   "batch": 1, "rows": N, "cols": K, "scale_layout": "row"},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": measured_traffic("gemv"), "kernel": "gemv kernel (oom_gemv_fp8, per-row scales)",
                     "algorithmic_bytes_per_step": float(bytes_call), "copy_gbs": copy_bandwidth(torch)},
    }
    if not args.no_cpu:
        xn = x.float().cpu().numpy()
        us, threads, n = cpu_baseline_gemv(xn, qs[0].cpu().numpy(), ss[0].cpu().numpy(), args.cpu_seconds)
        res["cpu_baseline"] = {"value": us, "unit": "us/call", "cores": threads, "kind": "port",
                               "sample": f"{n} calls of the same 4096x4096 GEMV, oracle restatement of the "
                                         f"reference's FP8 GEMV arithmetic, rows split over {threads} threads, on "
                                         f"{cpu_model()}"}
    return res


def cpu_baseline_attn(q, k, v, table, kv_len, H, Hkv, D, scale, budget_s):
    """The oracle's restatement of the reference attention on this host, one thread per
    KV head (each with its own copy of that head's pages), for about `budget_s` seconds.
    Returns (us_per_step, threads, steps)."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle

    G = H // Hkv
    heads = [(np.ascontiguousarray(q[g * G:(g + 1) * G]), np.ascontiguousarray(k[:, g:g + 1]),
              np.ascontiguousarray(v[:, g:g + 1])) for g in range(Hkv)]
    threads = max(1, min(Hkv, usable_cores()))

    def one(g):
        qg, kg, vg = heads[g]
        return oracle.attn_decode_paged(qg, kg, vg, table, 16, kv_len, G, 1, D, scale)

    t0 = time.perf_counter()
    steps = 0
    with ThreadPoolExecutor(threads) as pool:
        while True:
            list(pool.map(one, range(Hkv)))
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget_s and steps >= 2:
                break
    return el / steps * 1e6, threads, steps


def bench_attn(args):
    """Paged GQA decode attention, batch 1: 64 query heads, 8 KV heads, head_dim 128,
    32768 keys of bf16 K/V in 16-token pages in a seeded random page order, N(0, 1)
    q/K/V, all keys visible, bf16 out."""
    import numpy as np
    import torch

    import homelab_amd as hip

    H, Hkv, D, L, P = 64, 8, 128, 32768, 16
    n_pages = L // P
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    # three caches rotate between steps so K/V stream from HBM, not from the MALL
    caches = []
    for _ in range(3):
        k = torch.randn((n_pages, Hkv, P, D), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((n_pages, Hkv, P, D), generator=g, device="cuda").to(torch.bfloat16)
        table = torch.randperm(n_pages, generator=g, device="cuda").to(torch.int32)
        caches.append((k, v, table))
    q = torch.randn((H, D), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((H, D), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(hip.attn_decode_workspace_size(L, H, Hkv, D), dtype=torch.uint8, device="cuda")
    scale = 1.0 / D ** 0.5
    stream = torch.cuda.current_stream()

    def step(i):
        k, v, table = caches[i % 3]
        hip.attn_decode_paged(q, k, v, table, L, scale, out, ws, stream)

    for i in range(args.warmup):
        step(i)
    ms, timing = time_rounds(step, 0, args, stream, torch)
    bytes_step = 2 * L * Hkv * D * 2 + L // P * 4 + 2 * H * D * 2
    gbs = bytes_step / (ms * 1e-3) / 1e9
    res = {
        "metric": "GQA paged decode attention us/step + achieved HBM GB/s (% of MI355X peak), 1 GPU",
        "value": ms * 1e3, "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "timing": timing, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 K/V/q, fp32 softmax and accumulate, bf16 out", "data": "synthetic",
        "config": {"workload": "GQA decode attention, batch 1: 64 q heads, 8 KV heads, head_dim 128, 32768 keys, "
                               "bf16 KV in 16-token pages in random page order; 3 caches rotate past the MALL",
                   "heads": H, "kv_heads": Hkv, "head_dim": D, "kv_len": L, "page_size": P},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": measured_traffic("attn"), "kernel": "attn_decode_kernel (oom_attn_decode_paged)",
                     "algorithmic_bytes_per_step": bytes_step, "copy_gbs": copy_bandwidth(torch)},
    }
    if not args.no_cpu:
        kk, vv, tt = caches[0]
        k16 = kk.view(torch.int16).cpu().numpy().view(np.uint16)
        v16 = vv.view(torch.int16).cpu().numpy().view(np.uint16)
        q16 = q.view(torch.int16).cpu().numpy().view(np.uint16)
        us, threads, n = cpu_baseline_attn(q16, k16, v16, tt.cpu().numpy(), L, H, Hkv, D, scale, args.cpu_seconds)
        res["cpu_baseline"] = {"value": us, "unit": "us/step", "cores": threads, "kind": "port",
                               "sample": f"{n} runs of the same attention step, oracle restatement of the reference's "
                                         f"fp32 attention, one thread per KV head, on {cpu_model()}"}
    return res


def bench_turbo(args):
    """The product's own decode attention, batch 1: 24 query heads over 2 KV heads,
    head_dim 256, 32768 keys in a Turbo k8v6 cache (K rows 8-bit, V rows 6-bit Lloyd-Max
    codes over the rotated vector, fp16 block RMS scales), f32 q and out, all keys
    visible (mask of ones), through oom_attn_decode_turbo: q rotation, mask_compact, the
    flash-decode partials, their combine and the inverse rotation, all timed."""
    import numpy as np
    import torch

    import homelab_amd as hip

    H, Hkv, D, L, KB, VB = 24, 2, 256, 32768, 8, 6
    levels = torch.from_numpy(hip.kv_codebooks()).cuda()
    krb, vrb = hip.kv_row_bytes(D, KB), hip.kv_row_bytes(D, VB)
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    # twelve caches (30 MB each) rotate between steps so the rows stream from HBM, not the MALL
    copies = 12
    caches = []
    src = torch.empty((L, Hkv, D), dtype=torch.float32, device="cuda")
    for _ in range(copies):
        kc = torch.empty(L * Hkv * krb, dtype=torch.uint8, device="cuda")
        vc = torch.empty(L * Hkv * vrb, dtype=torch.uint8, device="cuda")
        src.normal_(generator=g)
        hip.kv_append(src, kc, 0, KB, levels)
        src.normal_(generator=g)
        hip.kv_append(src, vc, 0, VB, levels)
        caches.append((kc, vc))
    del src
    q = torch.randn((H, D), generator=g, device="cuda")
    mask = torch.ones(L, dtype=torch.uint8, device="cuda")
    out = torch.empty((H, D), dtype=torch.float32, device="cuda")
    ws = torch.zeros(hip.attn_decode_turbo_workspace_size(H, Hkv, D, L), dtype=torch.uint8, device="cuda")
    scale = 1.0 / 16.0
    stream = torch.cuda.current_stream()
    fn = hip.lib().oom_attn_decode_turbo
    cargs = [(hip._ptr(q), hip._ptr(kc), hip._ptr(vc), KB, VB, hip._ptr(levels), hip._ptr(mask), H, Hkv, D, L, scale,
              hip._ptr(out), hip._ptr(ws), ws.numel(), hip._stream(stream)) for kc, vc in caches]
    hip.attn_decode_turbo(q, caches[0][0], caches[0][1], KB, VB, levels, mask, Hkv, L, scale, out, ws, stream)

    def step(i):
        rc = fn(*cargs[i % copies])
        if rc:
            hip.check(rc)

    for i in range(args.warmup):
        step(i)
    ms, timing = time_rounds(step, 0, args, stream, torch)
    bytes_step = L * Hkv * (krb + vrb) + L + 2 * H * D * 4
    gbs = bytes_step / (ms * 1e-3) / 1e9
    res = {
        "metric": "Turbo k8v6 decode attention us/step + achieved HBM GB/s (% of MI355X peak), 1 GPU",
        "value": ms * 1e3, "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "timing": timing, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "k8v6 Lloyd-Max codes with fp16 scales, f32 q/softmax/accumulate/out", "data": "synthetic",
        "config": {"workload": "decode attention, batch 1: 24 q heads over 2 KV heads, head_dim 256, 32768 keys, "
                               "Turbo k8v6 rows of N(0,1) vectors, all keys visible; 12 caches rotate past the MALL",
                   "heads": H, "kv_heads": Hkv, "head_dim": D, "kv_len": L, "k_bits": KB, "v_bits": VB,
                   "row_bytes": [krb, vrb]},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": measured_traffic("turbo"), "kernel": "all kernels of oom_attn_decode_turbo (sum)",
                     "algorithmic_bytes_per_step": bytes_step, "copy_gbs": copy_bandwidth(torch)},
    }
    if not args.no_cpu:
        import oracle

        qn, kn, vn, mn = q.cpu().numpy(), caches[0][0].cpu().numpy(), caches[0][1].cpu().numpy(), mask.cpu().numpy()
        t0 = time.perf_counter()
        n = 0
        while True:
            oracle.attn_decode_turbo(qn, kn, vn, KB, VB, mn, H, Hkv, L, scale)
            n += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds and n >= 2:
                break
        res["cpu_baseline"] = {"value": el / n * 1e6, "unit": "us/step", "cores": 1, "kind": "port",
                               "sample": f"{n} runs of the same attention step, oracle restatement of the reference's "
                                         f"Turbo row decode and fp32 flash-decode arithmetic, one thread, on "
                                         f"{cpu_model()}"}
    return res


def cpu_baseline_layer(host_recs, shared_rec, rw_bits, gw_bits, geo, sgeo, E, k, T, budget_s=10.0):
    """The reference CPU path of a whole decode MoE layer (oracle restatement of
    crates/oominf-cpu): router GEMV over bf16 weights, top-k, plan, HostExperts for the
    routed experts and the shared expert, the shared gate GEMV, slot-order combine and the
    sigmoid-gated add, fresh activations each step, for about `budget_s` seconds.
    Returns (us_per_token, cores, steps)."""
    import numpy as np

    import oracle

    cores = usable_cores()
    rng = np.random.default_rng(6)
    t0 = time.perf_counter()
    steps = 0
    while True:
        x = oracle.bf16_to_f32(oracle.bf16_from_f32(rng.standard_normal((T, geo.hidden)).astype(np.float32)))
        logits = oracle.gemv_bf16(x, rw_bits)
        ids, w = oracle.router_topk(logits, k)
        experts, off, tok, slot = oracle.moe_plan(ids, E)
        jobs = [tok[off[i]:off[i + 1]] for i in range(len(experts))]
        y = oracle.host_experts(geo, [host_recs[e] for e in experts], jobs, x, cores)
        routed = oracle.moe_combine_slots(y, slot, w)
        shared = oracle.host_experts(sgeo, [shared_rec], [np.arange(T, dtype=np.int32)], x, cores)
        gate = oracle.gemv_bf16(x, gw_bits)
        oracle.moe_combine_shared(routed, shared, gate)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s and steps >= 3:
            break
    return el / steps / T * 1e6, cores, steps


def bench_layer(args, T, config):
    """A whole decode MoE layer per step through oom_moe_layer_decode_fp8: router GEMV over
    bf16 weights [128, 4096] from N(0, 0.02), top-8, the routed experts of the decode
    workload (hidden 4096, inter 1536, e4m3 128x128-block-scaled), one shared expert of the
    same geometry with a sigmoid gate over bf16 weights [4096], bf16 x from N(0, 1) fresh
    each step. Two sets of every weight alternate between steps so all of them stream
    from HBM."""
    import numpy as np
    import torch

    import homelab_amd as hip

    E, k, H, I, SI = 128, 8, 4096, 1536, 1536
    geo, sgeo = hip.record_geometry(H, I), hip.record_geometry(H, SI)
    stride, sstride = hip.record_stride(geo), hip.record_stride(sgeo)
    log(f"bench: layer T={T} E={E} k={k} H={H} I={I} shared inter {SI}; building 2 expert sets of "
        f"{E * stride / 1e9:.2f} GB")
    sets = [make_expert_set(E, geo, stride, 1234 + s, torch) for s in range(2)]
    addrs = [torch.tensor([b.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
             for b in sets]
    shared = make_expert_set(2, sgeo, sstride, 777, torch)
    saddrs = [torch.tensor([shared.data_ptr() + s * sstride], dtype=torch.int64, device="cuda") for s in range(2)]
    g = torch.Generator(device="cuda")
    g.manual_seed(98)
    rws = [(torch.randn((E, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16) for _ in range(2)]
    gws = [(torch.randn((1, H), generator=g, device="cuda") * 0.02).to(torch.bfloat16) for _ in range(2)]
    n = args.warmup + args.rounds * args.steps
    xs = torch.randn((n, T, H), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ids = torch.empty((n, T, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((n, T, k), dtype=torch.float32, device="cuda")
    ws = torch.zeros(hip.moe_layer_decode_fp8_workspace_size(T, E, k, geo, sgeo), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def step(i):
        s = i % 2
        hip.moe_layer_decode_fp8(xs[i], rws[s], addrs[s], k, geo, saddrs[s], sgeo, gws[s], ids[i], wts[i], out, ws,
                                 stream)

    for i in range(args.warmup):
        step(i)
    ms, timing = time_rounds(step, args.warmup, args, stream, torch)
    # algorithmic bytes: each distinct routed expert once, the shared expert, the router
    # and gate weights, x and out
    idn = ids[args.warmup:].cpu().numpy()
    distinct = np.array([len(np.unique(s_)) for s_ in idn])
    per_expert = 3 * H * I + 3 * (H // 128) * (I // 128) * 4
    per_shared = 3 * H * SI + 3 * (H // 128) * (SI // 128) * 4
    bytes_step = float(distinct.mean()) * per_expert + per_shared + (E + 1) * H * 2 + 2 * T * H * 2
    gbs = bytes_step / (ms * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": ms * 1e3 / T,
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "timing": timing,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 expert weights, bf16 router/gate weights and activations, fp32 accumulate",
        "data": "synthetic",
        "config": {"workload": f"whole decode MoE layer, batch {T}: bf16 router GEMV 128 x 4096, 128 experts top-8, "
                               "hidden 4096, inter 1536, plus one shared expert (inter 1536) with a sigmoid gate; "
                               "e4m3 128x128-block-scaled expert weights from N(0,0.02), bf16 x fresh each step; "
                               "2 sets of all weights alternate past the MALL",
                   "batch": T, "experts": E, "top_k": k, "hidden": H, "inter": I, "shared_inter": SI,
                   "distinct_experts_per_step": float(distinct.mean())},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": measured_traffic(config),
                     "kernel": "oom_moe_layer_decode_fp8 step: the router GEMV, then one decode kernel with the "
                               "shared expert, its gate logit and the gated add inside it "
                               f"({'moe_decode_fused_kernel' if T == 1 else 'moe_batch_kernel'})",
                     "algorithmic_bytes_per_step": bytes_step, "copy_gbs": copy_bandwidth(torch)},
    }
    if not args.no_cpu:
        import oracle

        host = sets[0].cpu().numpy()
        ogeo, osgeo = oracle.record_geometry(H, I), oracle.record_geometry(H, SI)
        rw_bits = rws[0].view(torch.int16).cpu().numpy().view(np.uint16)
        gw_bits = gws[0].view(torch.int16).cpu().numpy().view(np.uint16)
        us, cores, nsteps = cpu_baseline_layer([host[e] for e in range(E)], shared[0].cpu().numpy(), rw_bits, gw_bits,
                                               ogeo, osgeo, E, k, T, args.cpu_seconds)
        res["cpu_baseline"] = {"value": us, "unit": "us/token", "cores": cores, "kind": "port",
                               "sample": f"{nsteps} steps of the same batch-{T} whole decode MoE layer (fresh x), "
                                         f"oracle restatement of the reference CPU path on {cpu_model()}"}
    return res


def make_nvfp4_set(E, geo, stride, seed, torch):
    """[E, stride] uint8 NVFP4 records: random code bytes, scale bytes in [0x28, 0x50)
    (positive e4m3 values of about 2^-2 .. 2^2), weight_scale_2 in [0.01, 0.03)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    buf = torch.zeros((E, stride), dtype=torch.uint8, device="cuda")
    H, I = geo.hidden, geo.inter
    for wo, so, n, k in [(geo.gate_weight, geo.gate_scale, I, H), (geo.up_weight, geo.up_scale, I, H),
                         (geo.down_weight, geo.down_scale, H, I)]:
        buf[:, wo:wo + n * k // 2] = torch.randint(0, 256, (E, n * k // 2), generator=g, device="cuda",
                                                   dtype=torch.uint8)
        buf[:, so:so + n * k // 16] = torch.randint(0x28, 0x50, (E, n * k // 16), generator=g, device="cuda",
                                                    dtype=torch.uint8)
    scal = torch.zeros((E, 64), dtype=torch.float32, device="cuda")
    for i in range(3):
        scal[:, geo.scale2[i]] = 0.01 + 0.02 * torch.rand((E,), generator=g, device="cuda")
    buf[:, :256] = scal.view(torch.uint8)
    return buf


def bench_nvfp4_prefill(args):
    """The routed experts of one prefill group over NVFP4 records on the bf16 matrix cores,
    the reference's tiled path (crates/oominf-models-qwen/src/moe.rs:746-758): gate and up
    with oom_moe_tiled_nvfp4, oom_moe_swiglu_range, down with oom_moe_tiled_nvfp4, and the
    slot-order combine. 2048 tokens, 512 experts top-10, hidden 2560, inter 640 (about 40
    assignments an expert: the reference's prefill_throughput shape,
    crates/oominf-cuda/tests/moe_tiled.rs:229-246). Routing and the plan are made once
    before the timed steps; activations f32 x N(0, 1)."""
    import numpy as np
    import torch

    import homelab_amd as hip

    T, E, k, H, I = 2048, 512, 10, 2560, 640
    exact = args.prefill_precision == "exact"
    prec = hip.EXPERT_EXACT if exact else hip.EXPERT_BF16
    geo = hip.nvfp4_geometry(H, I)
    stride = hip.nvfp4_stride(geo)
    log(f"bench: nvfp4 prefill T={T} E={E} k={k} H={H} I={I} {args.prefill_precision}; "
        f"building {E * stride / 1e9:.2f} GB of records")
    recset = make_nvfp4_set(E, geo, stride, 1357, torch)
    addrs = torch.tensor([recset.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(71)
    logits = torch.randn((T, E), generator=g, device="cuda")
    x = torch.randn((T, H), generator=g, device="cuda")
    A = T * k
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, k), dtype=torch.float32, device="cuda")
    hip.router_topk(logits, ids, wts, k)
    plan = torch.empty(hip.moe_plan_size(T, E, k), dtype=torch.int32, device="cuda")
    recs = torch.empty(E, dtype=torch.int64, device="cuda")
    hip.moe_plan(ids, E, addrs, plan, recs)
    torch.cuda.synchronize()
    hp = plan.cpu().numpy()
    n_e = int(hp[0])
    off_h = hp[1 + E:1 + E + n_e + 1]
    max_n = int(np.diff(off_h).max())
    off = plan[1 + E:]
    assign_tok = plan[1 + E + E + 1:1 + E + E + 1 + A]
    slot_assign = plan[1 + E + E + 1 + A:1 + E + E + 1 + 2 * A].view(T, k)
    gbuf = torch.empty((A, I), dtype=torch.float32, device="cuda")
    ubuf = torch.empty_like(gbuf)
    hbuf = torch.empty_like(gbuf)
    ybuf = torch.empty((A, H), dtype=torch.float32, device="cuda")
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream()

    def step():
        hip.moe_tiled_nvfp4(recs, off, assign_tok, n_e, max_n, x, gbuf, I, H, geo.gate_weight, geo.gate_scale,
                            geo.scale2[0], prec, stream)
        hip.moe_tiled_nvfp4(recs, off, assign_tok, n_e, max_n, x, ubuf, I, H, geo.up_weight, geo.up_scale,
                            geo.scale2[1], prec, stream)
        hip.moe_swiglu_range(gbuf, ubuf, hbuf, 0, A * I, stream)
        hip.moe_tiled_nvfp4(recs, off, None, n_e, max_n, hbuf, ybuf, H, I, geo.down_weight, geo.down_scale,
                            geo.scale2[2], prec, stream)
        hip.moe_combine_slots(ybuf, slot_assign, wts, out, stream)

    for _ in range(args.warmup):
        step()
    ms, timing = time_rounds(lambda i: step(), 0, args, stream, torch)
    per_expert = 3 * H * I // 2 + 3 * H * I // 16 + 12
    bytes_step = n_e * per_expert + T * H * 4 + T * H * 2
    terms = 3 if exact else 1
    flops = 2.0 * A * 3 * H * I * terms  # the matrix-core work: three projections, one pass a term
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = bytes_step / (ms * 1e-3) / 1e9
    res = {
        "metric": "MoE NVFP4 prefill (tiled, bf16 matrix cores) us/step + roofline fraction, 1 GPU",
        "value": ms * 1e3, "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "timing": timing, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "nvfp4 weights decoded exactly to bf16, f32 activations as " +
                 ("three exact bf16 terms" if exact else "bf16") + ", fp32 accumulate",
        "data": "synthetic",
        "config": {"workload": "routed experts of a 2048-token prefill group over nvfp4-modelopt-g16 records: 512 "
                               "experts top-10, hidden 2560, inter 640, random codes and scales, N(0,1) logits and "
                               "x; gate, up, SwiGLU, down, slot-order combine (routing made once)",
                   "tokens": T, "experts": E, "top_k": k, "hidden": H, "inter": I, "distinct_experts": n_e,
                   "max_per_expert": max_n, "expert_precision": args.prefill_precision,
                   "tokens_per_s": T / (ms * 1e-3), "hbm_gbs": gbs},
        "roofline": ({"bound": "mfma", "achieved": tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                      "frac": tflops / PEAK_BF16_TFLOPS} if exact else
                     {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS})
        | {"traffic": measured_traffic("nvfp4_prefill"), "kernel": "moe_tiled_nvfp4_wide_kernel (three launches a step)",
           "algorithmic_bytes_per_step": bytes_step, "matrix_flops_per_step": flops},
    }
    if not args.no_cpu:
        import oracle

        # the oracle's single-thread restatement of the same three projections over a sample
        # of 8 experts' assignments, scaled to the step's n_e experts
        host = recset.cpu().numpy()
        ids_h, wh = ids.cpu().numpy(), wts.cpu().numpy()
        xs = x.cpu().numpy()
        S = 8
        sexp = hp[1:1 + n_e][:S]
        soff = off_h[:S + 1] - off_h[0]
        stok = hp[1 + E + E + 1:1 + E + E + 1 + A][off_h[0]:off_h[S]]
        srecs = [host[int(e)] for e in sexp]
        t0 = time.perf_counter()
        reps = 0
        while True:
            gg = oracle.moe_tiled_nvfp4(srecs, soff, stok, xs, I, H, geo.gate_weight, geo.gate_scale, geo.scale2[0],
                                        terms)
            uu = oracle.moe_tiled_nvfp4(srecs, soff, stok, xs, I, H, geo.up_weight, geo.up_scale, geo.scale2[1],
                                        terms)
            hh = (gg / (1.0 + np.exp(-gg)) * uu).astype(np.float32)
            oracle.moe_tiled_nvfp4(srecs, soff, None, hh, H, I, geo.down_weight, geo.down_scale, geo.scale2[2], terms)
            reps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds and reps >= 1:
                break
        per = el / reps * (A / max(1, int(soff[-1])))
        res["cpu_baseline"] = {"value": per * 1e6, "unit": "us/step", "cores": 1, "kind": "port",
                               "sample": f"{reps} runs of gate, up, SwiGLU and down for 8 experts' "
                                         f"{int(soff[-1])} assignments with the oracle's restatement of the "
                                         f"reference's tiled arithmetic, scaled to the step's {A} assignments, "
                                         f"on {cpu_model()}"}
        del ids_h, wh
    return res


def bench_bf16(args):
    """The routed experts over bf16 records (the format's unquantised `bf16` layout) at the
    FP8 decode shape: 128 experts, 8 picked per step, hidden 4096, inter 1536, batch 1, bf16
    x; a step is oom_moe_gate_up_bf16, oom_moe_down_bf16 and oom_moe_combine_slots over a
    plan built beforehand for every step (seeded picks, different experts each step). Two
    sets of 128 records (2 x 4.8 GB) alternate so weights stream from HBM."""
    import numpy as np
    import torch

    import homelab_amd as hip

    T, E, k, H, I = 1, 128, 8, 4096, 1536
    geo = hip.bf16_geometry(H, I)
    stride = (geo.down_weight + H * I * 2 + 4095) // 4096 * 4096
    log(f"bench: bf16-record experts T={T} E={E} k={k} H={H} I={I}; building 2 sets of {E * stride / 1e9:.2f} GB")
    g = torch.Generator(device="cuda")
    g.manual_seed(123)
    sets = []
    for s_ in range(2):
        buf = torch.empty((E, stride), dtype=torch.uint8, device="cuda")
        for e in range(E):
            for off_, n in [(geo.gate_weight, I * H), (geo.up_weight, I * H), (geo.down_weight, H * I)]:
                w = (torch.randn(n, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
                buf[e, off_:off_ + 2 * n] = w.view(torch.uint8)
        sets.append(buf)
    n = args.warmup + args.rounds * args.steps
    rng = np.random.default_rng(5)
    picks = np.stack([np.sort(rng.choice(E, size=k, replace=False)) for _ in range(n)])
    recs = torch.tensor([[sets[i % 2].data_ptr() + int(e) * stride for e in picks[i]] for i in range(n)],
                        dtype=torch.int64, device="cuda")
    off = torch.arange(k + 1, dtype=torch.int32, device="cuda")
    tok = torch.zeros(k, dtype=torch.int32, device="cuda")
    slot = torch.arange(k, dtype=torch.int32, device="cuda").reshape(1, k)
    wts = torch.full((1, k), 1.0 / k, dtype=torch.float32, device="cuda")
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    h = torch.empty((k, I), dtype=torch.float32, device="cuda")
    y = torch.empty((k, H), dtype=torch.float32, device="cuda")
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream()

    def step(i):
        hip.moe_gate_up_bf16(recs[i], off, tok, k, x, h, geo, stream)
        hip.moe_down_bf16(recs[i], off, k, h, y, geo, stream)
        hip.moe_combine_slots(y, slot, wts, out, stream)

    for i in range(args.warmup):
        step(i)
    ms, timing = time_rounds(step, args.warmup, args, stream, torch)
    bytes_step = k * 3 * H * I * 2 + 2 * T * H * 2
    gbs = bytes_step / (ms * 1e-3) / 1e9
    return {
        "metric": "bf16-record routed experts us/token + achieved HBM GB/s (% of MI355X peak), 1 GPU",
        "value": ms * 1e3 / T, "unit": "us/token", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "timing": timing, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 weights and x, fp32 accumulate", "data": "synthetic",
        "config": {"workload": "routed experts over bf16 records, batch 1: 8 of 128 experts a step, hidden 4096, "
                               "inter 1536, bf16 N(0,0.02) weights; 2 record sets alternate past the MALL",
                   "batch": T, "experts": E, "picked": k, "hidden": H, "inter": I},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": measured_traffic("bf16"), "kernel": "moe_gate_up_bf16_kernel + moe_down_bf16_kernel",
                     "algorithmic_bytes_per_step": float(bytes_step)},
    }


def bench_nvfp4(args):
    """One routed MoE decode step over NVFP4 (nvfp4-modelopt-g16) records at the released
    model's routed geometry: 512 experts, top-10, hidden 2560, inter 640, batch 1, fresh
    N(0, 1) logits each step, bf16 x (oom_moe_decode_nvfp4)."""
    import numpy as np
    import torch

    import homelab_amd as hip

    T, E, k, H, I = 1, 512, 10, 2560, 640
    geo = hip.nvfp4_geometry(H, I)
    stride = hip.nvfp4_stride(geo)
    log(f"bench: nvfp4 decode T={T} E={E} k={k} H={H} I={I}; building 2 expert sets of {E * stride / 1e9:.2f} GB")
    sets = [make_nvfp4_set(E, geo, stride, 2468 + s, torch) for s in range(2)]
    addrs = [torch.tensor([b.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
             for b in sets]
    n = args.warmup + args.rounds * args.steps
    g = torch.Generator(device="cuda")
    g.manual_seed(97)
    logits = torch.randn((n, T, E), generator=g, device="cuda").contiguous()
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ids = torch.empty((n, T, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((n, T, k), dtype=torch.float32, device="cuda")
    ws = torch.zeros(hip.moe_decode_nvfp4_workspace_size(T, E, k, geo), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def step(i):
        hip.moe_decode_nvfp4(logits[i], x, addrs[i % 2], k, geo, ids[i], wts[i], out, ws, stream)

    for i in range(args.warmup):
        step(i)
    ms, timing = time_rounds(step, args.warmup, args, stream, torch)
    idn = ids[args.warmup:].cpu().numpy()
    distinct = float(np.mean([len(np.unique(s_)) for s_ in idn]))
    per_expert = 3 * H * I // 2 + 3 * H * I // 16 + 12  # codes, scale bytes, the three scale_2 floats
    bytes_step = distinct * per_expert + 2 * T * H * 2
    gbs = bytes_step / (ms * 1e-3) / 1e9
    res = {
        "metric": "MoE NVFP4 decode step us/token + achieved HBM GB/s (% of MI355X peak), 1 GPU",
        "value": ms * 1e3 / T, "unit": "us/token", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "timing": timing, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "nvfp4 (e2m1 + e4m3 group-16 scales) weights, bf16 activations, fp32 accumulate",
        "data": "synthetic",
        "config": {"workload": "MoE FFN decode step over nvfp4-modelopt-g16 records, batch 1: 512 experts top-10, "
                               "hidden 2560, inter 640, random codes and scales, fresh N(0,1) logits; 2 expert sets "
                               "alternate past the MALL",
                   "batch": T, "experts": E, "top_k": k, "hidden": H, "inter": I,
                   "distinct_experts_per_step": distinct},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": measured_traffic("nvfp4"),
                     "kernel": "moe_decode_nvfp4_1p_kernel (oom_moe_decode_nvfp4, one launch for one token)",
                     "algorithmic_bytes_per_step": bytes_step, "copy_gbs": copy_bandwidth(torch)},
    }
    if not args.no_cpu:
        import oracle

        host = sets[0].cpu().numpy()
        ogeo = oracle.nvfp4_geometry(H, I)
        recs = [host[e] for e in range(E)]
        rng = np.random.default_rng(8)
        xs = x.float().cpu().numpy()
        t0 = time.perf_counter()
        reps = 0
        while True:
            oracle.moe_decode_nvfp4(rng.standard_normal((T, E)).astype(np.float32), xs, recs, k, ogeo)
            reps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds and reps >= 3:
                break
        res["cpu_baseline"] = {"value": el / reps / T * 1e6, "unit": "us/token", "cores": 1, "kind": "port",
                               "sample": f"{reps} steps of the same decode (fresh logits), the oracle's scalar "
                                         f"restatement of the reference's nvfp4_rows_scalar path, one thread, on "
                                         f"{cpu_model()}"}
    return res


PEAK_FP8_TFLOPS = 5000.0


def bench_prefill(args):
    """MoE prefill step: 2048 tokens, hidden 4096, 128 experts top-8 with Zipf(1.1)-biased
    N(0, 1) router logits, e4m3 128x128-block-scaled expert weights (gate/up 1536 x 4096,
    down 4096 x 1536) from N(0, 0.02), bf16 x from N(0, 1); per-token e4m3 activations,
    gate/up grouped GEMM on FP8 MFMA, SiLU*mul, down over h kept at fp32 precision as two
    bf16 terms on bf16 MFMA (the reference's default ExpertPrecision::Exact;
    --prefill-precision bf16 rounds h to bf16 for one pass), weighted combine
    (oom_moe_prefill_fp8)."""
    import numpy as np
    import torch

    import homelab_amd as hip

    T, E, k, H, I = 2048, 128, 8, 4096, 1536
    geo = hip.record_geometry(H, I)
    stride = hip.record_stride(geo)
    log(f"bench: prefill T={T} E={E} k={k} H={H} I={I}; building an expert set of {E * stride / 1e9:.2f} GB")
    rec = make_expert_set(E, geo, stride, 4321, torch)
    addrs = torch.tensor([rec.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(17)
    n = args.warmup + args.rounds * args.steps
    bias = torch.from_numpy(zipf_bias(E, 1.1, 7)).cuda()
    logits = (torch.randn((n, T, E), generator=g, device="cuda") + bias).contiguous()
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ids = torch.empty((n, T, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((n, T, k), dtype=torch.float32, device="cuda")
    ws = torch.zeros(hip.moe_prefill_fp8_workspace_size(T, E, k, geo), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    prec = hip.EXPERT_EXACT if args.prefill_precision == "exact" else hip.EXPERT_BF16
    terms = 2 if prec == hip.EXPERT_EXACT else 1

    def step(i):
        hip.moe_prefill_fp8(logits[i], x, addrs, k, geo, ids[i], wts[i], out, ws, stream, precision=prec)

    for i in range(args.warmup):
        step(i)
    ms, timing = time_rounds(step, args.warmup, args, stream, torch)
    idn = ids[args.warmup:].cpu().numpy()
    distinct = float(np.mean([len(np.unique(s_)) for s_ in idn]))
    per_expert = 3 * H * I + 3 * (H // 128) * (I // 128) * 4
    bytes_step = distinct * per_expert + T * H * 2 * 2
    flops = 2.0 * T * k * 3 * H * I
    gbs = bytes_step / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    # gate/up (2/3 of the flops) run on FP8 MFMA, down on bf16 MFMA over h's bf16 terms
    # (issued once a term): the step's matrix-core time at peak, and the rate that implies
    t_peak = (2.0 / 3.0) * flops / (PEAK_FP8_TFLOPS * 1e12) + terms * (1.0 / 3.0) * flops / (PEAK_BF16_TFLOPS * 1e12)
    peak_mix = flops / t_peak / 1e12
    res = {
        "metric": "MoE FP8 prefill step us/step + achieved HBM GB/s and FP8 MFMA TFLOP/s (% of MI355X peak), 1 GPU",
        "value": ms * 1e3, "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "timing": timing, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8-e4m3 weights; e4m3 activations (gate/up), h as " + ("two bf16 terms" if terms == 2 else "bf16")
                 + " (down); fp32 accumulate, bf16 out",
        "data": "synthetic",
        "config": {"workload": "MoE prefill grouped GEMM: 2048 tokens x hidden 4096, 128 experts top-8 with Zipf(1.1) "
                               "biased logits, inter 1536, e4m3 128x128-block-scaled weights, per-token e4m3 "
                               "activations", "tokens": T, "experts": E, "top_k": k, "hidden": H, "inter": I,
                   "distinct_experts_per_step": distinct, "tokens_per_s": T / (ms * 1e-3),
                   "expert_precision": args.prefill_precision},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": measured_traffic("prefill"), "kernel": "oom_moe_prefill_fp8 step (all its kernels)",
                     "algorithmic_bytes_per_step": bytes_step, "copy_gbs": copy_bandwidth(torch)},
        "mfma": {"achieved": tflops, "peak": peak_mix, "unit": "TFLOP/s", "frac": tflops / peak_mix,
                 "flops_per_step": flops,
                 "peak_note": f"gate/up at the FP8 peak, down's {terms} bf16 pass(es) at the bf16 peak"},
    }
    if not args.no_cpu:
        import oracle

        host = rec.cpu().numpy()
        ogeo = oracle.record_geometry(H, I)
        sample = 64
        lg = logits[0, :sample].cpu().numpy()
        xs = x[:sample].float().cpu().numpy()
        cores = usable_cores()
        t0 = time.perf_counter()
        reps = 0
        while True:
            ids_h, w_h = oracle.router_topk(lg, k)
            experts, off, tok, slot = oracle.moe_plan(ids_h, E)
            jobs = [tok[off[i]:off[i + 1]] for i in range(len(experts))]
            y = oracle.host_experts(ogeo, [host[e] for e in experts], jobs, xs, cores)
            oracle.moe_combine_slots(y, slot, w_h)
            reps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds and reps >= 1:
                break
        res["cpu_baseline"] = {"value": el / reps / sample * T * 1e6, "unit": "us/step", "cores": cores, "kind": "port",
                               "sample": f"{reps} runs of the first {sample} tokens of a step (router, plan, "
                                         f"HostExperts, combine: the reference CPU path, oracle restatement), scaled "
                                         f"to {T} tokens, on {cpu_model()}"}
    return res



PEAK_PCIE_GBS = 64.0  # PCIe 5.0 x16, one direction


def bench_offload(args):
    """The batch-1 FP8 decode step with every expert in the host tier: per step the routed
    experts' records (8 x 18.9 MB) copy from pinned host memory into device slots on a copy
    queue, double-buffered so step i+1's copies run beside step i's compute, ordered with
    events (oom_copy_records_to_device, oom_event_record, oom_stream_wait_event). The
    routing of every step is computed on the device before the timed region."""
    import numpy as np
    import torch

    import homelab_amd as hip

    T, E, k, H, I = 1, 128, 8, 4096, 1536
    geo = hip.record_geometry(H, I)
    stride = hip.record_stride(geo)
    steps = min(args.steps, 50)
    warmup = min(args.warmup, 5)
    n = warmup + args.rounds * steps
    log(f"bench: offload decode T={T} E={E} k={k} H={H} I={I}; {E * stride / 1e9:.2f} GB of records in pinned host memory")
    dev_set = make_expert_set(E, geo, stride, 1234, torch)
    host = hip.PinnedHost(E * stride)
    host.array()[:] = dev_set.reshape(-1).cpu().numpy()
    del dev_set
    torch.cuda.empty_cache()
    g = torch.Generator(device="cuda")
    g.manual_seed(99)
    logits = torch.randn((n, T, E), generator=g, device="cuda").contiguous()
    ids = torch.empty((n, T, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((n, T, k), dtype=torch.float32, device="cuda")
    for i in range(n):
        hip.router_topk(logits[i], ids[i], wts[i], k)
    routed = ids.cpu().numpy()
    slots = [torch.empty((k, stride), dtype=torch.uint8, device="cuda") for _ in range(2)]
    dst = [[b.data_ptr() + j * stride for j in range(k)] for b in slots]
    tables = []
    for i in range(n):
        t = np.full(E, dst[i % 2][0], dtype=np.int64)
        for j, e in enumerate(routed[i, 0]):
            t[e] = dst[i % 2][j]
        tables.append(torch.from_numpy(t).cuda())
    x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(T, E, k, geo), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    q = hip.CopyQueue()
    copied = [hip.Event() for _ in range(n)]
    computed = [hip.Event() for _ in range(n)]

    def stage(i):
        if i >= 2:
            computed[i - 2].wait_on(q)  # the slots' previous reader is done
        q.copy_records(dst[i % 2], [host.ptr + int(e) * stride for e in routed[i, 0]], stride)
        copied[i].record(q)

    def run(lo, hi):
        stage(lo)
        for i in range(lo, hi):
            if i + 1 < hi:
                stage(i + 1)
            copied[i].wait_on(stream)
            hip.moe_decode_fp8(logits[i], x, tables[i], k, geo, ids[i], wts[i], out, ws, stream)
            computed[i].record(stream)

    run(0, warmup)
    per = []
    for r in range(args.rounds):
        torch.cuda.synchronize()
        q.sync()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        run(warmup + r * steps, warmup + (r + 1) * steps)
        end.record(stream)
        torch.cuda.synchronize()
        q.sync()
        per.append(start.elapsed_time(end) / steps)
    ms = sorted(per)[len(per) // 2]
    timing = {"rounds": len(per), "steps_per_round": steps, "round_ms": [round(v, 6) for v in per],
              "spread": (max(per) - min(per)) / ms}
    h2d = k * stride / (ms * 1e-3) / 1e9
    for ev in copied + computed:
        ev.close()
    q.close()
    host.close()
    return {
        "metric": "MoE FP8 decode step with host-tier experts: us/token + host-to-device GB/s, 1 GPU",
        "value": ms * 1e3 / T, "unit": "us/token", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "timing": timing, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8-e4m3 weights, bf16 activations, fp32 accumulate", "data": "synthetic",
        "config": {"workload": "MoE FFN decode step, batch 1: 128 experts top-8, hidden 4096, inter 1536, all "
                               "records in pinned host memory; the 8 routed records copy to device slots each step "
                               "on a copy queue, double-buffered beside compute",
                   "batch": T, "experts": E, "top_k": k, "hidden": H, "inter": I},
        "roofline": {"bound": "pcie", "achieved": h2d, "peak": PEAK_PCIE_GBS, "unit": "GB/s",
                     "frac": h2d / PEAK_PCIE_GBS, "traffic": None,
                     "kernel": "host-to-device copies of the routed records (oom_copy_records_to_device)",
                     "algorithmic_bytes_per_step": float(k * stride)},
    }

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--rounds", type=int, default=5,
                    help="timed rounds of --steps launches each; the value is the median round")
    ap.add_argument("--config", default="decode1", choices=["decode1", "decode16", "layer1", "layer16", "nvfp4", "offload", "attn",
                                                            "turbo", "prefill", "nvfp4-prefill", "gemv", "copy", "bf16"])
    ap.add_argument("--prefill-precision", default="exact", choices=["exact", "bf16"],
                    help="activation precision of the prefill's down projection (the reference's ExpertPrecision)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build measures one MI355X (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    # Every config launches on a stream of its own (default priority), not on the null
    # stream: a launch on HIP's null stream carries its implicit synchronisation with every
    # other stream, measured at ~2.7 us per launch (a 5.0 us GEMV timed 7.8 us a call there).
    launch = torch.cuda.Stream()
    with torch.cuda.stream(launch):
        res = run_config(args, torch)
    print(json.dumps(res), flush=True)


def run_config(args, torch):
    if args.config == "copy":
        # the PMC calibration run: copies of exactly 1 GiB, nothing else on the GPU
        gbs = copy_bandwidth(torch, 1 << 30, args.steps)
        res = {"metric": "device copy GB/s (read + write)", "value": gbs, "unit": "GB/s", "bytes_per_copy": 1 << 30,
               "copies": args.steps + 1}
    elif args.config == "attn":
        res = bench_attn(args)
    elif args.config == "turbo":
        res = bench_turbo(args)
    elif args.config == "nvfp4-prefill":
        res = bench_nvfp4_prefill(args)
    elif args.config == "gemv":
        res = bench_gemv(args)
    elif args.config == "prefill":
        res = bench_prefill(args)
    elif args.config == "decode1":
        res = bench_decode(args, 1, None, args.config)
    elif args.config == "offload":
        res = bench_offload(args)
    elif args.config == "nvfp4":
        res = bench_nvfp4(args)
    elif args.config == "bf16":
        res = bench_bf16(args)
    elif args.config in ("layer1", "layer16"):
        res = bench_layer(args, 1 if args.config == "layer1" else 16, args.config)
    else:
        res = bench_decode(args, 16, 1.1, args.config)
    return res


if __name__ == "__main__":
    main()
