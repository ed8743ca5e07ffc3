#!/usr/bin/env python3
"""Benchmark: HAT-S x4 on a 512x512 fp32 input, single pass, on one MI355X.

One "step" is one whole forward (src/gpu.rs:759-803 `Gpu::forward`, minus the
host copies): input [3][512][512] already in HBM, output [3][2048][2048] written
to HBM. `value` is output megapixels per second over exactly --steps steps,
bracketed by device synchronisations.

Also reported on the same JSON line:
  * roofline: the shifted-window attention kernel (the metric's second half,
    "window-attn % FP32-MFMA peak"), algorithmic FLOPs per launch
    4 * T * 256 * C (QK^T + PV, head_dim unpadded) over its mean launch time,
    measured with HIP events on the launch stream in a second pass of --steps
    steps; peak = 157.3 TFLOP/s (MI355X dense FP32 MFMA);
  * norm_roofline: the standalone LayerNorm kernel against HBM peak (8 TB/s),
    8*C bytes per token over its mean launch time (the other LayerNorms run in
    GEMM and conv epilogues);
  * kernels: the same per-kernel event times for every kernel of the forward;
  * cpu_baseline: the CPU oracle (a C restatement of the reference's src/cpu.rs,
    kind "port") timed on this host's cores on a bounded sample (one HAT-S x4
    forward at 128x128, i.e. 1/16 of the metric's pixels), in output Mpx/s;
  * wall_ms_incl_pcie: one forward including the H2D input and D2H output copies.
"""
import argparse
import json
import os
import sys
import tempfile
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "hat-rs_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

METRIC = "output Mpx/s HAT-S x4 512x512 fp32 (1 GPU); window-attn % FP32-MFMA peak"
PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense FP32 matrix
PEAK_HBM = 8000.0       # GB/s


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--size", type=int, default=512, help="input side (square)")
    ap.add_argument("--variant", default="hat-s")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-size", type=int, default=128)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(every GPU box here has one GPU; sharding by strips of window rows is designed, not built)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import hat_amd

    if not hat_amd.gpu_available():
        print("bench.py: no GPU / HIP runtime", file=sys.stderr)
        sys.exit(1)

    h = w = args.size
    scale = 4
    td = tempfile.mkdtemp()
    wpath = os.path.join(td, f"{args.variant}_x4_seed1.safetensors")
    hat_amd.generate_weights(wpath, args.variant, scale, 1)
    W = hat_amd.Weights(wpath)
    be = hat_amd.Backend(W)
    img = np.random.default_rng(1).random((3, h, w), dtype=np.float32)
    out_host = np.empty((3, h * scale, w * scale), dtype=np.float32)
    d_in = hat_amd.DeviceBuffer(img.nbytes)
    d_out = hat_amd.DeviceBuffer(out_host.nbytes)
    d_in.upload(img)
    log(f"bench: {args.variant} x{scale} {h}x{w} on {hat_amd.device_name()} "
        f"({hat_amd.device_cu_count()} CUs)")

    for _ in range(args.warmup):
        be.forward_device(h, w, d_in.ptr, d_out.ptr)
    be.synchronize()
    hat_amd.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        be.forward_device(h, w, d_in.ptr, d_out.ptr)
    be.synchronize()
    hat_amd.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    out_px = h * scale * w * scale
    value = out_px / 1e6 / (ms / 1e3)
    log(f"bench: {ms:.2f} ms/step, {value:.2f} output Mpx/s")
    d_out.download(out_host)
    assert np.isfinite(out_host).all()

    # Per-kernel HIP-event times over a second pass of the same steps.
    hat_amd.profile_begin()
    for _ in range(args.steps):
        be.forward_device(h, w, d_in.ptr, d_out.ptr)
    be.synchronize()
    stats = hat_amd.profile_end()
    kernels = {k: {"launches": n, "total_ms": round(t, 4), "mean_ms": round(t / n, 5)}
               for k, (n, t) in sorted(stats.items(), key=lambda kv: -kv[1][1])}

    T = h * w
    C = W.embed
    attn_name = "hat_attn_sw_d24" if W.head_dim == 24 else "hat_attn_sw_d30"
    n_a, t_a = stats[attn_name]
    attn_ms = t_a / n_a
    attn_flop = 4.0 * T * 256 * C
    achieved = attn_flop / (attn_ms / 1e3) / 1e12
    roofline = {"kernel": attn_name, "bound": "mfma", "achieved": round(achieved, 3),
                "peak": PEAK_FP32_MFMA, "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA, 4),
                "flop_per_launch": attn_flop, "mean_launch_ms": round(attn_ms, 5), "traffic": None}

    # HBM reference: the library's plain copy kernel over 1 GiB (read + write),
    # timed with events; rocprof counter runs of this script also see it, which
    # is what scales their FETCH_SIZE / WRITE_SIZE readings to bytes.
    nb = 1 << 30
    c_src = hat_amd.DeviceBuffer(nb)
    c_dst = hat_amd.DeviceBuffer(nb)
    hat_amd.device_copy(c_dst, c_src, nb)
    hat_amd.synchronize()
    hat_amd.profile_begin()
    for _ in range(3):
        hat_amd.device_copy(c_dst, c_src, nb)
    hat_amd.synchronize()
    cstat = hat_amd.profile_end()["hat_copy"]
    copy_gbps = 2 * nb / (cstat[1] / cstat[0] / 1e3) / 1e9
    c_src.free()
    c_dst.free()

    # The standalone LayerNorm (the forward's one norm kernel outside a GEMM or
    # conv epilogue) against HBM: 8*C bytes per token (read x, write y) + the
    # 8*C bytes of weight and bias.
    norm = None
    if "hat_layernorm" in stats:
        n_l, t_l = stats["hat_layernorm"]
        ln_ms = t_l / n_l
        ln_bytes = 8.0 * C * T + 8.0 * C
        gbps = ln_bytes / (ln_ms / 1e3) / 1e9
        norm = {"kernel": "hat_layernorm", "bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM,
                "unit": "GB/s", "frac": round(gbps / PEAK_HBM, 4), "bytes_per_launch": ln_bytes,
                "mean_launch_ms": round(ln_ms, 5)}

    traffic_file = os.path.join(REPO, "profiles", "traffic_hat_attn_sw_d24_hats512.json")
    if os.path.exists(traffic_file) and attn_name == "hat_attn_sw_d24" and h == 512:
        with open(traffic_file) as f:
            roofline["traffic"] = json.load(f)["bytes_per_launch"]

    # One forward with the PCIe copies, as the reference's Backend::forward does.
    t2 = time.perf_counter()
    be.forward(h, w, img)
    wall_ms = (time.perf_counter() - t2) * 1e3

    cpu = None
    if not args.no_cpu:
        import oracle
        threads = min(16, os.cpu_count() or 1)
        oracle.set_threads(threads)
        cs = args.cpu_size
        cimg = np.random.default_rng(2).random((3, cs, cs), dtype=np.float32)
        M = oracle.OracleModel(wpath)
        log(f"bench: CPU oracle HAT-S x4 {cs}x{cs} on {threads} threads ...")
        tc = time.perf_counter()
        M.forward(cs, cs, cimg)
        cpu_s = time.perf_counter() - tc
        cpu = {"value": round((cs * scale) ** 2 / 1e6 / cpu_s, 5), "unit": "output Mpx/s",
               "cores": threads, "kind": "port",
               "sample": f"one {args.variant} x4 forward at {cs}x{cs} (output {cs*scale}x{cs*scale}), "
                         f"{cpu_s:.2f} s"}
        log(f"bench: CPU {cpu_s:.2f} s -> {cpu['value']} output Mpx/s")

    line = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "output Mpx/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (uniform [0,1] input, seeded N(0,0.02) weights)",
        "config": {"workload": f"{args.variant} x4 {h}x{w} fp32 single-pass forward",
                   "input": f"{h}x{w}x3", "output": f"{h*scale}x{w*scale}x3",
                   "weights": "seeded, tools/convert.py format", "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "norm_roofline": norm,
        "cpu_baseline": cpu,
        "wall_ms_incl_pcie": round(wall_ms, 3),
        "copy_kernel_gbps": round(copy_gbps, 1),
        "acts_gib": round(be.acts_bytes() / 2**30, 3),
        "weights_mib": round(be.weight_bytes() / 2**20, 2),
        "device": hat_amd.device_name(),
        "kernels": kernels,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
