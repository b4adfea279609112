"""Per-wave phase timeline of the one-launch decode kernels, from a profiling build.

    python stamps.py --build                 # here (CPU): homelab_amd/_build_stamps/liboom_hip_stamps.so
    python stamps.py decode1 [--calls 40]    # on the GPU: the FP8 decode step, batch 1
    python stamps.py nvfp4 [--calls 40]      # on the GPU: the NVFP4 decode step, batch 1
    python stamps.py decode16 [--calls 40]   # on the GPU: the FP8 decode step, batch 16 (Zipf 1.1 routing)

The profiling build compiles every kernel with -DOOM_STAMPS: the one-launch decode kernels
then record the device's 100 MHz real-time clock per wave at their phase boundaries into a
buffer handed over by oom_debug_set_stamps (a symbol of that build only). This script loads
that library in place of liboom_hip.so, runs the bench workload of the config (bench.py's
expert sets and inputs: two sets alternate, fresh logits each call), stamps the last
`--calls` calls after a warm-up and prints, per point, the distribution over every wave of
every call of (stamp - the call's first wave start) in microseconds, then the per-call
spans. The stamps add a few instructions and one store per wave per point: a stamped call
runs slightly slower than the default build's.
"""
import argparse
import ctypes
import os
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
STAMPS_DIR = os.path.join(ROOT, "homelab_amd", "_build_stamps")
STAMPS_LIB = os.path.join(STAMPS_DIR, "liboom_hip_stamps.so")
POINTS = 8  # words per wave (STAMP_POINTS of homelab_amd/csrc/stream.hpp)

NAMES = {
    "decode1": ["start", "routed and planned", "gate/up done", "barrier released", "slot's h loaded",
                "tile rows done", "combined, stored"],
    "nvfp4": ["start", "routed (wave 0)", "x staged", "gate/up done", "barrier released", "h staged",
              "first tile combined", "end"],
    "decode16": ["start", "routed and planned", "gate/up done", "barrier 1 released", "first run's h staged",
                 "down tiles done", "combined, stored"],
}


# the point whose per-block distribution is broken down by XCD (hardware id in the last point)
WHERE_POINT = {"decode1": 2, "decode16": 2}


def build_stamps():
    from homelab_amd import build as b

    return b.build(verbose=True, build_dir=STAMPS_DIR, lib=STAMPS_LIB, defines=("OOM_STAMPS",))


def workload(config, torch, hip, bench):
    """(step(i), waves per block of the config's kernel, the buffers to keep alive) of the
    config's bench workload."""
    g = torch.Generator(device="cuda")
    if config == "decode16":
        # the bench's batch-16 workload: Zipf(1.1)-biased logits, two expert sets alternating
        E, k, H, I, T = 128, 8, 4096, 1536, 16
        geo = hip.record_geometry(H, I)
        stride = hip.record_stride(geo)
        sets = [bench.make_expert_set(E, geo, stride, 1234 + s, torch) for s in range(2)]
        g.manual_seed(99)
        ws = torch.zeros(hip.moe_decode_fp8_workspace_size(T, E, k, geo), dtype=torch.uint8, device="cuda")
        addrs = [torch.tensor([b.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
                 for b in sets]
        bias = torch.from_numpy(bench.zipf_bias(E, 1.1, 7)).cuda()
        logits = (torch.randn((256, T, E), generator=g, device="cuda") + bias).contiguous()
        x = torch.randn((T, H), generator=g, device="cuda").to(torch.bfloat16)
        out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
        w = torch.empty((T, k), dtype=torch.float32, device="cuda")

        def step16(i):
            hip.moe_decode_fp8(logits[i % 256], x, addrs[i % 2], k, geo, ids, w, out, ws)

        return step16, 8, (sets, addrs)
    if config == "decode1":
        E, k, H, I = 128, 8, 4096, 1536
        geo = hip.record_geometry(H, I)
        stride = hip.record_stride(geo)
        sets = [bench.make_expert_set(E, geo, stride, 1234 + s, torch) for s in range(2)]
        g.manual_seed(99)
        ws = torch.zeros(hip.moe_decode_fp8_workspace_size(1, E, k, geo), dtype=torch.uint8, device="cuda")
        step_fn = hip.moe_decode_fp8
        waves = 8
    else:
        E, k, H, I = 512, 10, 2560, 640
        geo = hip.nvfp4_geometry(H, I)
        stride = hip.nvfp4_stride(geo)
        sets = [bench.make_nvfp4_set(E, geo, stride, 2468 + s, torch) for s in range(2)]
        g.manual_seed(97)
        ws = torch.zeros(hip.moe_decode_nvfp4_workspace_size(1, E, k, geo), dtype=torch.uint8, device="cuda")
        step_fn = hip.moe_decode_nvfp4
        waves = 4
    addrs = [torch.tensor([b.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
             for b in sets]
    logits = torch.randn((256, 1, E), generator=g, device="cuda").contiguous()
    x = torch.randn((1, H), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
    ids = torch.empty((1, k), dtype=torch.int32, device="cuda")
    w = torch.empty((1, k), dtype=torch.float32, device="cuda")

    def step(i):
        step_fn(logits[i % 256], x, addrs[i % 2], k, geo, ids, w, out, ws)

    return step, waves, (sets, addrs)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("config", nargs="?", choices=["decode1", "nvfp4", "decode16"])
    ap.add_argument("--build", action="store_true", help="build the profiling library (no GPU needed)")
    ap.add_argument("--calls", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=20)
    args = ap.parse_args()
    if args.build:
        build_stamps()
        if not args.config:
            return 0
    if not args.config:
        ap.error("name a config (decode1, nvfp4 or decode16) or --build")
    if not os.path.exists(STAMPS_LIB):
        sys.exit(f"{STAMPS_LIB} is missing: run `python stamps.py --build` first")
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    import homelab_amd as hip

    hip.LIB_PATH = STAMPS_LIB  # before the first call loads a library
    import bench

    lib = hip.lib()
    lib.oom_debug_set_stamps.argtypes = [ctypes.c_void_p]
    step, waves, keep = workload(args.config, torch, hip, bench)
    blocks = 4096  # above any resident grid of these kernels
    buf = torch.zeros(blocks * waves * POINTS, dtype=torch.int64, device="cuda")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    lib.oom_debug_set_stamps(ctypes.c_void_p(buf.data_ptr()))
    rel, spans, per_block = [], [], []
    npt = len(NAMES[args.config])
    try:
        for i in range(args.warmup, args.warmup + args.calls):
            buf.zero_()
            torch.cuda.synchronize()
            step(i)
            torch.cuda.synchronize()
            raw = buf.cpu().numpy().reshape(blocks, waves, POINTS)
            launched = raw[:, 0, 0] > 0
            raw = raw[launched]
            t = raw.reshape(-1, POINTS).astype(np.float64)
            t0 = t[:, 0].min()
            r = (t[:, :npt] - t0) * 0.01  # 100 MHz ticks -> us
            r[t[:, :npt] == 0] = np.nan  # a point the wave never passed (a block with no output tile)
            rel.append(r)
            spans.append(np.nanmax(r[:, npt - 1]))
            if WHERE_POINT.get(args.config) is not None:
                # per block: the last wave's stamp of the phase-end point, and where block ran
                done = np.nanmax(r[:, WHERE_POINT[args.config]].reshape(-1, waves), axis=1)
                where = raw[:, 0, POINTS - 1].astype(np.uint64)
                per_block.append((done, (where >> np.uint64(32)) & np.uint64(15),
                                  (where >> np.uint64(8)) & np.uint64(0xff)))
    finally:
        lib.oom_debug_set_stamps(None)
    status = hip.status()
    r = np.concatenate(rel)
    print(f"{args.config}: {args.calls} stamped calls, {r.shape[0] // args.calls} waves a call, status {status}")
    print("point                   min      p10      p50      p90      max   (us after the call's first wave start)")
    for j, name in enumerate(NAMES[args.config]):
        v = r[:, j][~np.isnan(r[:, j])]
        print(f"{name:<20} {v.min():8.2f} {np.percentile(v, 10):8.2f} {np.median(v):8.2f} {np.percentile(v, 90):8.2f}"
              f" {v.max():8.2f}   ({v.size // args.calls} waves a call)")
    print(f"call span (last wave's end): median {np.median(spans):.2f} us, min {min(spans):.2f}, max {max(spans):.2f}")
    if per_block:
        # the phase end per block (its last wave), by the XCD the block ran on
        name = NAMES[args.config][WHERE_POINT[args.config]]
        done = np.concatenate([d for d, _, _ in per_block])
        xcc = np.concatenate([x for _, x, _ in per_block]).astype(int)
        print(f"per block, {name} (its last wave): p10 {np.percentile(done, 10):.2f}, p50 {np.median(done):.2f}, "
              f"p90 {np.percentile(done, 90):.2f}, max {done.max():.2f}")
        for x in range(int(xcc.max()) + 1):
            v = done[xcc == x]
            if v.size:
                print(f"  XCD {x}: {v.size // args.calls:4d} blocks a call, p50 {np.median(v):.2f}, "
                      f"p90 {np.percentile(v, 90):.2f}, max {v.max():.2f}")
        # does the same (XCD, SE/CU) finish last call after call?
        last = [(int(x[np.argmax(d)]), int(c[np.argmax(d)])) for d, x, c in per_block]
        print("  last block of each call (XCD, hw id bits 8..15):", " ".join(f"{x}/{c:02x}" for x, c in last))
    del keep
    return 0


if __name__ == "__main__":
    sys.exit(main())
