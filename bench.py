"""Headline benchmark: SigLIP2-so400m Q8_0 vision tower, batch 32 x 729
patches (27x27 grid, GEMM M = 23328), probe pooling, one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 32]
                    [--cpu-images 3] [--no-cpu]

A step = one encode of the whole batch with the pixels already resident in
HBM.  Prints ONE JSON line.  `roofline` reports the dominant kernel (the
Q8_0 x Q8_1 MFMA GEMM): algorithmic int8 ops (2*M*N*K_logical, padding not
counted) over the GEMM launch durations measured with HIP events on the
encoder's stream during the timed steps, against MI355X's dense int8 peak.
`cpu_baseline` times the CPU oracle (this repository's C restatement of
ggml's CPU Q8_0 path) on a bounded sample of the same workload.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hbd-siglip2.cpp_amd"))

INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, published
METRIC = "images/sec SigLIP2 vision Q8_0 @729 patches; MMQ int8 TOPS % of peak"
KERNEL = ("k_gemm (Q8_0 x Q8_1 GEMM, persistent 256x128 tiles: int8 quants and scales by LDS DMA, "
          "v_mfma_i32_32x32x32_i8 block dots, dx*dw scale tile on v_mfma_f32_32x32x8_f16, one "
          "convert + fma per element and block; priced against the int8 peak)")
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_vision_b32_traffic.json")


def traffic_per_launch():
    """HBM bytes per GEMM launch of this workload, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (calibrated on a copy kernel);
    None when not measured for this kernel."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        return int(json.load(f)["bytes_per_launch"])


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--cpu-images", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run one device-to-device copy of BYTES (a plain copy kernel "
                         "for calibrating HBM byte counters) and exit")
    ap.add_argument("--preproc", action="store_true",
                    help="instead of the tower: time the NaFlex front end (GPU resize + "
                         "patchify of a batch of RGB images) and print its own JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on one GPU: the library has no multi-GPU path (the tower "
              "shards as independent data-parallel replicas; see the design notes)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.copy_probe:
        n = args.copy_probe // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n * 4}), flush=True)
        return

    import s2x
    from s2x import synth

    if args.preproc:
        bench_preproc(args, np, torch, s2x)
        return

    cfg = synth.SO400M_VISION
    B, gh, gw = args.batch, 27, 27
    n_pos = gh * gw
    log(f"bench: generating so400m weights (seeded), batch {B} x {n_pos}")
    hm = synth.vision_model(cfg, seed=0)
    v = ctypes.c_void_p()
    s2x.call("s2x_vision_create", ctypes.byref(hm.struct), ctypes.byref(v))
    stream = torch.cuda.ExternalStream  # noqa: F841 (the encoder owns its stream)
    px = synth.pixels(B, n_pos, seed=1234)
    pd = torch.from_numpy(px).to("cuda:0")
    out = torch.empty((B, cfg.hidden), dtype=torch.float32, device="cuda:0")

    def step():
        s2x.call("s2x_vision_encode_batch_dev", v, ctypes.c_void_p(pd.data_ptr()), B, gh, gw,
                 s2x.POOL_PROBE, ctypes.c_void_p(out.data_ptr()))

    def sync():
        # the encoder's stream: a zero-length stats query synchronises it
        s2x.call("s2x_vision_gemm_stats", v, None, None, None, 0)
        torch.cuda.synchronize()

    log("bench: warmup")
    for _ in range(args.warmup):
        step()
    sync()
    s2x.call("s2x_vision_gemm_stats", v, None, None, None, 1)
    s2x.call("s2x_vision_gemm_timing", v, 1)
    log(f"bench: timing {args.steps} steps")
    sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    sync()
    t1 = time.perf_counter()
    ms = ctypes.c_double()
    ops = ctypes.c_double()
    launches = ctypes.c_int64()
    s2x.call("s2x_vision_gemm_stats", v, ctypes.byref(ms), ctypes.byref(ops),
             ctypes.byref(launches), 1)
    s2x.call("s2x_vision_gemm_timing", v, 0)
    emb = out.cpu().numpy()
    assert np.isfinite(emb).all()
    s2x.lib.s2x_vision_destroy(v)

    ms_step = (t1 - t0) * 1000.0 / args.steps
    ips = B / (ms_step / 1000.0)
    gemm_tops = ops.value / (ms.value / 1000.0) / 1e12
    avg_launch_ms = ms.value / max(1, launches.value)
    log(f"bench: {ms_step:.2f} ms/step, {ips:.1f} images/s, GEMM {gemm_tops:.1f} TOPS over "
        f"{launches.value} launches (avg {avg_launch_ms * 1000:.1f} us), "
        f"GEMM share of step {ms.value / args.steps / ms_step * 100:.1f}%")

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pyoracle
        om = pyoracle.vision_model(hm)
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        log(f"bench: CPU baseline (oracle, {threads} threads, {args.cpu_images} image(s))")
        c0 = time.perf_counter()
        for i in range(args.cpu_images):
            pyoracle.vision_encode(om, px[i * n_pos:(i + 1) * n_pos], gh, gw, pooling=1,
                                   nthreads=threads)
        c1 = time.perf_counter()
        cpu = {"value": round(args.cpu_images / (c1 - c0), 4), "unit": "images/s",
               "cores": threads, "kind": "port",
               "sample": f"{args.cpu_images} image(s) of the same 27x27 so400m probe-pooled "
                         f"workload, batch 1, {c1 - c0:.1f} s"}

    rec = {
        "metric": METRIC,
        "value": round(ips, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) Q8_0 weights, uniform[-1,1] patches)",
        "config": {"workload": "SigLIP2-so400m vision tower, 27 blocks, Q8_0, batch 32 x 729 "
                               "patches (27x27), probe pooling", "global_batch": B,
                   "seq_len": n_pos, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 2),
                     "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tops / INT8_PEAK_TOPS, 4),
                     "traffic": traffic_per_launch(),
                     "kernel": KERNEL,
                     "avg_launch_ms": round(avg_launch_ms, 4),
                     "launches": int(launches.value)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


def bench_preproc(args, np, torch, s2x):
    """The NaFlex front end on its own: B RGB images of 640 x 480 resized to
    at most 729 patches of 16 x 16 and patchified (s2x_nf_preprocess_rgb_batch_dev:
    one launch per pass for the batch, images already in HBM).  Roofline:
    HBM, algorithmic bytes = the u8 images read + the f32 patch rows written."""
    B, H, W, MP, P = args.batch, 480, 640, 729, 16
    rng = np.random.default_rng(7)
    imgs = torch.from_numpy(rng.integers(0, 256, (B, H, W, 3), dtype=np.uint8)).to("cuda:0")
    th, tw = ctypes.c_int32(), ctypes.c_int32()
    s2x.call("s2x_nf_target_size", H, W, P, MP, ctypes.byref(th), ctypes.byref(tw))
    n_rows = (th.value // P) * (tw.value // P)
    feat = 3 * P * P
    out = torch.empty((B, n_rows * feat), dtype=torch.float32, device="cuda:0")
    wsb = B * s2x.lib.s2x_nf_workspace_size(H, W, P, MP)
    ws = torch.empty((wsb,), dtype=torch.uint8, device="cuda:0")
    mean = np.array([0.5, 0.5, 0.5], np.float32)
    std = np.array([0.5, 0.5, 0.5], np.float32)
    stream = torch.cuda.current_stream().cuda_stream
    nh, nw = ctypes.c_int32(), ctypes.c_int32()

    def step():
        s2x.call("s2x_nf_preprocess_rgb_batch_dev", ctypes.c_void_p(imgs.data_ptr()), B, H, W, MP,
                 P, ctypes.c_float(1.0 / 255.0), mean.ctypes.data, std.ctypes.data,
                 ctypes.c_void_p(out.data_ptr()), n_rows * feat, ctypes.byref(nh),
                 ctypes.byref(nw), ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(wsb),
                 ctypes.c_void_p(stream))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    gpu_ms = e0.elapsed_time(e1) / args.steps
    ms_step = (t1 - t0) * 1000.0 / args.steps
    ips = B / (ms_step / 1000.0)
    alg_bytes = B * (H * W * 3 + n_rows * feat * 4)
    gbs = alg_bytes / (gpu_ms / 1000.0) / 1e9
    log(f"preproc: {ms_step:.3f} ms/step wall, {gpu_ms:.3f} ms/step GPU, {ips:.0f} images/s, "
        f"{gbs:.0f} GB/s algorithmic")
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pyoracle
        host_imgs = [im.cpu().numpy() for im in imgs[:8]]
        done = 0
        c0 = time.perf_counter()
        while time.perf_counter() - c0 < 10.0:  # a bounded ~10 s sample
            pyoracle.nf_preprocess_rgb(host_imgs[done % len(host_imgs)], MP, p=P, fused=1)
            done += 1
        c1 = time.perf_counter()
        cpu = {"value": round(done / (c1 - c0), 2), "unit": "images/s", "cores": 1,
               "kind": "port", "sample": f"{done} images (8 distinct) of the same 640x480 -> "
                                         f"{n_rows}-patch workload, {c1 - c0:.1f} s"}
    rec = {
        "metric": f"images/sec NaFlex preprocessing 640x480 RGB -> {n_rows} patches of 16x16",
        "value": round(ips, 1), "unit": "images/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded uniform u8 RGB images)",
        "config": {"workload": f"NaFlex front end, batch {B} x 640x480 RGB, max 729 patches",
                   "global_batch": B, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(gbs / 8000.0, 4), "traffic": None,
                     "kernel": "k_nf_vpass + k_nf_hpass (one launch each per batch)",
                     "avg_launch_ms": round(gpu_ms / 2, 4), "launches": 2 * args.steps},
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
