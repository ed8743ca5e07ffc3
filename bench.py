#!/usr/bin/env python3
"""Benchmark: HAT-S x4 on a 512x512 fp32 input, single pass, on one MI355X.

One "step" is one whole forward (src/gpu.rs:759-803 `Gpu::forward`, minus the
host copies): input [3][512][512] already in HBM, output [3][2048][2048] written
to HBM. `value` is output megapixels per second over exactly --steps steps,
bracketed by device synchronisations. Weights: seeded N(0, 0.02) (libhat's
generator, seed 1); input: uniform [0, 1) (numpy PCG64, seed 1).

Also reported on the same JSON line:
  * step_ms: min / median of --steps further forwards, each synchronised on
    its own (the reference's bench.rs:145-164 statistics);
  * roofline: the shifted-window attention kernel (the metric's second half,
    "window-attn % FP32-MFMA peak"), algorithmic FLOPs per launch
    4 * T * 256 * C (QK^T + PV, head_dim unpadded) over its mean launch time,
    measured with HIP events on the launch stream over a pass of --steps
    forwards; peak = 157.3 TFLOP/s (MI355X dense FP32 MFMA); traffic = HBM
    bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs;
    bf16_executed: the BF16-MFMA work the kernel executes for it (six bf16
    products per fp32 product, padding included; committed counter run)
    against the dense BF16 peak (2.5 PFLOP/s);
  * norm_roofline: the standalone LayerNorm kernel against HBM peak (8 TB/s);
  * kernels: the same per-kernel event times for every kernel of the forward;
  * pcie: min / median wall time of a forward from and to host memory (the
    reference's Backend::forward shape), never the headline;
  * host_peak_rss_mib: the process's peak resident set (VmHWM) after the
    metric configuration's forwards, as the reference's bench reports it;
  * configs: benchmark configurations 2-5 of the plan as extra figures - the
    SW-MSA op (128 x 128, C = 180, shift 0 and 8) and the OCAB op with their
    head_dim-30 attention kernels' fractions of peak, HAT x4 at 256 x 256 and
    HAT-L x4 at 512 x 512 (with its measured device working set);
  * cpu_baseline: the CPU oracle (a C restatement of the reference's src/cpu.rs,
    kind "port") on this host: benchmark config 1 (one HAT-S x4 forward at
    64 x 64) min of 3 after a warm-up, in output Mpx/s, plus the config 2 and 3
    ops; the threads used, nproc and the CPU model are stated.
"""
import argparse
import json
import os
import statistics
import sys
import tempfile
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "hat-rs_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

METRIC = "output Mpx/s HAT-S x4 512x512 fp32 (1 GPU); window-attn % FP32-MFMA peak"
PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense FP32 matrix
PEAK_BF16_MFMA = 2500.0  # TFLOP/s, MI355X dense BF16 matrix
PEAK_HBM = 8000.0       # GB/s
WEIGHT_SEED = 1
INPUT_SEED = 1
# The box allots 16 host cores to one GPU, whatever nproc reports.
CPU_SHARE = 16


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_peak_rss_mib():
    """The process's peak resident set (VmHWM), as the reference's bench reports it
    beside the device working set (examples/bench.rs:85-100)."""
    try:
        with open("/proc/self/status") as f:
            for line in f:
                if line.startswith("VmHWM:"):
                    return round(int(line.split()[1]) / 1024.0, 1)
    except (OSError, ValueError, IndexError):
        pass
    return None


def stats_ms(samples):
    return {"min": round(min(samples), 4), "median": round(statistics.median(samples), 4),
            "n": len(samples)}


def timed_steps(fn, sync, n):
    out = []
    for _ in range(n):
        t = time.perf_counter()
        fn()
        sync()
        out.append((time.perf_counter() - t) * 1e3)
    return out


def extra_configs(hat_amd, np, td, steps):
    """Benchmark configurations 2-5 (the plan's cfg2/cfg3 ops, HAT 256, HAT-L 512)."""
    out = {}
    rng = np.random.default_rng(2024)
    c, hh, ww, heads = 180, 128, 128, 6
    T = hh * ww
    x = rng.standard_normal((T, c), dtype=np.float32)
    sw = [rng.standard_normal(s, dtype=np.float32) * 0.02 for s in
          ((3 * c, c), (3 * c,), (c, c), (c,), (961, heads))]
    for shift in (0, 8):
        _, ms, ams = hat_amd.op_swmsa(x, hh, ww, c, heads, shift, *sw, iters=max(steps, 5))
        flop = 4.0 * T * 256 * c
        tf = flop / (ams / 1e3) / 1e12
        out[f"cfg2_swmsa_shift{shift}"] = {
            "workload": "SW-MSA op 128x128 C=180 6 heads (qkv + attention + proj)",
            "op_ms": round(ms, 4), "attn_kernel": "hat_attnx_swp_d30", "attn_ms": round(ams, 4),
            "attn_flop": flop, "attn_tflops": round(tf, 2), "attn_frac": round(tf / PEAK_FP32_MFMA, 4)}
    shapes = [(c,), (c,), (3 * c, c), (3 * c,), (c, c), (c,), (1521, heads), (c,), (c,),
              (2 * c, c), (2 * c,), (c, 2 * c), (c,)]
    ws = [rng.standard_normal(s, dtype=np.float32) * 0.02 for s in shapes]
    ws[0][:] = 1.0
    ws[1][:] = 0.0
    ws[7][:] = 1.0
    ws[8][:] = 0.0
    _, ms, ams = hat_amd.op_ocab(x, hh, ww, c, heads, 2, ws, iters=max(steps, 5))
    flop = 4.0 * T * 576 * c
    tf = flop / (ams / 1e3) / 1e12
    out["cfg3_ocab"] = {
        "workload": "OCAB op 128x128 C=180 576 keys (norm1 + qkv + attention + proj + MLP)",
        "op_ms": round(ms, 4), "attn_kernel": "hat_attnx_oca_d30", "attn_ms": round(ams, 4),
        "attn_flop": flop, "attn_tflops": round(tf, 2), "attn_frac": round(tf / PEAK_FP32_MFMA, 4)}

    for name, variant, size, seed in (("cfg4_hat_x4_256", "hat", 256, 4), ("cfg5_hatl_x4_512", "hat-l", 512, 5)):
        wp = os.path.join(td, f"{variant}_x4_s{seed}.safetensors")
        hat_amd.generate_weights(wp, variant, 4, seed)
        W = hat_amd.Weights(wp)
        free0 = hat_amd.device_mem_info()[0]
        be = hat_amd.Backend(W)
        img = np.random.default_rng(seed).random((3, size, size), dtype=np.float32)
        d_in = hat_amd.DeviceBuffer(img.nbytes)
        d_out = hat_amd.DeviceBuffer(3 * size * size * 16 * 4)
        d_in.upload(img)
        free1 = hat_amd.device_mem_info()[0]
        be.forward_device(size, size, d_in.ptr, d_out.ptr)
        be.synchronize()
        free2 = hat_amd.device_mem_info()[0]
        t = timed_steps(lambda: be.forward_device(size, size, d_in.ptr, d_out.ptr), be.synchronize,
                        max(3, min(steps, 5)))
        s = stats_ms(t)
        out[name] = {
            "workload": f"{variant} x4 {size}x{size} fp32 single-pass forward",
            "ms": s, "output_mpx_s_at_median": round((4 * size) ** 2 / 1e6 / (s["median"] / 1e3), 3),
            "weights_mib": round(be.weight_bytes() / 2**20, 1),
            "per_plan_gib": round(be.acts_bytes() / 2**30, 3),
            # device memory the backend holds, by hipMemGetInfo: the weights
            # (uploaded when the backend is made) plus the plan's buffers (the
            # first forward), without the benchmark's own input/output buffers
            "device_working_set_gib": round((free0 - free2 - (d_in.nbytes + d_out.nbytes)) / 2**30, 3),
            "plan_alloc_gib": round((free1 - free2) / 2**30, 3),
            "weight_seed": seed, "input_seed": seed}
        log(f"bench: {name}: median {s['median']:.2f} ms")
        d_in.free()
        d_out.free()
        be.close()
    return out


def cpu_baseline(np, wpath, scale):
    import oracle
    threads = max(1, min(CPU_SHARE, os.cpu_count() or 1))
    oracle.set_threads(threads)
    M = oracle.OracleModel(wpath)
    cs = 64
    img = np.random.default_rng(64).random((3, cs, cs), dtype=np.float32)
    log(f"bench: CPU oracle HAT-S x4 {cs}x{cs} on {threads} threads ...")
    M.forward(cs, cs, img)  # warm-up
    t = []
    for _ in range(3):
        tc = time.perf_counter()
        M.forward(cs, cs, img)
        t.append(time.perf_counter() - tc)
    best = min(t)
    rng = np.random.default_rng(2024)
    c, hh, ww = 180, 128, 128
    x = rng.standard_normal((hh * ww, c), dtype=np.float32)
    sw = [rng.standard_normal(s, dtype=np.float32) * 0.02 for s in
          ((3 * c, c), (3 * c,), (c, c), (c,), (961, 6))]
    ops = {}
    for shift in (0, 8):
        oracle.swmsa_op(x, hh, ww, c, 6, shift, *sw)
        tt = []
        for _ in range(3):
            tc = time.perf_counter()
            oracle.swmsa_op(x, hh, ww, c, 6, shift, *sw)
            tt.append((time.perf_counter() - tc) * 1e3)
        ops[f"cfg2_swmsa_shift{shift}_ms"] = round(min(tt), 2)
    shapes = [(c,), (c,), (3 * c, c), (3 * c,), (c, c), (c,), (1521, 6), (c,), (c,),
              (2 * c, c), (2 * c,), (c, 2 * c), (c,)]
    ws = [rng.standard_normal(s, dtype=np.float32) * 0.02 for s in shapes]
    oracle.ocab_op(x, hh, ww, c, 6, 2, ws)
    tt = []
    for _ in range(3):
        tc = time.perf_counter()
        oracle.ocab_op(x, hh, ww, c, 6, 2, ws)
        tt.append((time.perf_counter() - tc) * 1e3)
    ops["cfg3_ocab_ms"] = round(min(tt), 2)
    out = {"value": round((cs * scale) ** 2 / 1e6 / best, 5), "unit": "output Mpx/s",
           "cores": threads, "kind": "port",
           "sample": f"benchmark config 1: one HAT-S x4 forward at {cs}x{cs} (output {cs*scale}x{cs*scale}, "
                     f"1/64 of the metric's pixels), min of 3 after a warm-up: {best:.3f} s",
           "nproc": os.cpu_count(), "cpu_model": cpu_model(), "ops_min_ms": ops}
    log(f"bench: CPU {best:.3f} s -> {out['value']} output Mpx/s; ops {ops}")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--size", type=int, default=512, help="input side (square)")
    ap.add_argument("--variant", default="hat-s")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip benchmark configurations 2-5")
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
    wpath = os.path.join(td, f"{args.variant}_x4_seed{WEIGHT_SEED}.safetensors")
    hat_amd.generate_weights(wpath, args.variant, scale, WEIGHT_SEED)
    W = hat_amd.Weights(wpath)
    be = hat_amd.Backend(W)
    img = np.random.default_rng(INPUT_SEED).random((3, h, w), dtype=np.float32)
    out_host = np.empty((3, h * scale, w * scale), dtype=np.float32)
    d_in = hat_amd.DeviceBuffer(img.nbytes)
    d_out = hat_amd.DeviceBuffer(out_host.nbytes)
    d_in.upload(img)
    log(f"bench: {args.variant} x{scale} {h}x{w} on {hat_amd.device_name()} "
        f"({hat_amd.device_cu_count()} CUs)")

    def step():
        be.forward_device(h, w, d_in.ptr, d_out.ptr)

    for _ in range(args.warmup):
        step()
    be.synchronize()
    hat_amd.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    be.synchronize()
    hat_amd.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    out_px = h * scale * w * scale
    value = out_px / 1e6 / (ms / 1e3)
    log(f"bench: {ms:.2f} ms/step, {value:.2f} output Mpx/s")
    d_out.download(out_host)
    assert np.isfinite(out_host).all()

    step_ms = stats_ms(timed_steps(step, be.synchronize, args.steps))

    # Per-kernel HIP-event times over a further pass of the same steps.
    hat_amd.profile_begin()
    for _ in range(args.steps):
        step()
    be.synchronize()
    stats = hat_amd.profile_end()
    kernels = {k: {"launches": n, "total_ms": round(t, 4), "mean_ms": round(t / n, 5)}
               for k, (n, t) in sorted(stats.items(), key=lambda kv: -kv[1][1])}

    T = h * w
    C = W.embed
    attn_name = "hat_attnx_sw_d24" if W.head_dim == 24 else "hat_attnx_swp_d30"
    n_a, t_a = stats[attn_name]
    attn_ms = t_a / n_a
    attn_flop = 4.0 * T * 256 * C
    achieved = attn_flop / (attn_ms / 1e3) / 1e12
    roofline = {"kernel": attn_name, "bound": "mfma",
                "work": "fp32-equivalent: algorithmic fp32 FLOPs (head_dim unpadded) against the FP32-MFMA peak; "
                        "the kernel computes them on the BF16 MFMA path as six bf16 products each "
                        "(bf16_executed below is its utilisation of that path)",
                "achieved": round(achieved, 3),
                "peak": PEAK_FP32_MFMA, "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA, 4),
                "flop_per_launch": attn_flop, "mean_launch_ms": round(attn_ms, 5), "traffic": None}
    # The kernel computes on the BF16 matrix path (six bf16 products per fp32
    # product): the work it executes there, from the committed counter run,
    # against the dense BF16 peak.
    traffic_file = os.path.join(REPO, "profiles", "traffic_%s_hats512.json" % attn_name)
    if os.path.exists(traffic_file) and h == 512 and args.variant == "hat-s":
        with open(traffic_file) as f:
            tr = json.load(f)
        roofline["traffic"] = tr["bytes_per_launch"]
        bf16 = tr["bf16_gflop_executed"] / attn_ms  # GFLOP per ms = TFLOP/s
        roofline["bf16_executed"] = {"gflop_per_launch": tr["bf16_gflop_executed"], "achieved": round(bf16, 1),
                                     "peak": PEAK_BF16_MFMA, "unit": "TFLOP/s",
                                     "frac": round(bf16 / PEAK_BF16_MFMA, 4)}

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

    # Forwards from and to host memory, as the reference's Backend::forward does
    # (through the C ABI's caller-allocated output, reused across calls).
    be.forward(h, w, img, out_host)
    pcie = stats_ms(timed_steps(lambda: be.forward(h, w, img, out_host), lambda: None, max(5, args.steps)))
    pcie["output_mpx_s_at_median"] = round(out_px / 1e6 / (pcie["median"] / 1e3), 3)
    acts_gib = round(be.acts_bytes() / 2**30, 3)
    weights_mib = round(be.weight_bytes() / 2**20, 2)
    # before the extra configurations and the CPU oracle, which hold their own buffers
    rss_mib = host_peak_rss_mib()
    d_in.free()
    d_out.free()
    be.close()

    configs = None
    if not args.no_extra:
        configs = extra_configs(hat_amd, np, td, args.steps)

    cpu = None if args.no_cpu else cpu_baseline(np, wpath, scale)

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
        "data": "synthetic (uniform [0,1) input, seeded N(0,0.02) weights)",
        "config": {"workload": f"{args.variant} x4 {h}x{w} fp32 single-pass forward",
                   "input": f"{h}x{w}x3", "output": f"{h*scale}x{w*scale}x3",
                   "weights": "seeded, tools/convert.py format", "parallelism": "none (1 GPU)",
                   "seeds": {"weights": WEIGHT_SEED, "input": INPUT_SEED}},
        "step_ms": step_ms,
        "roofline": roofline,
        "norm_roofline": norm,
        "cpu_baseline": cpu,
        "pcie": pcie,
        "copy_kernel_gbps": round(copy_gbps, 1),
        "acts_gib": acts_gib,
        "weights_mib": weights_mib,
        "host_peak_rss_mib": rss_mib,
        "device": hat_amd.device_name(),
        "configs": configs,
        "kernels": kernels,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
