"""Forward-pass throughput of a KataGo network on one MI355X: evals/s at a fixed batch.

Default workload: b18c384nbt (18 nested-bottleneck blocks, 384 trunk channels, 192 inner), fp16 GEMM operands
with float accumulate, batch 32, 19x19, seeded synthetic weights and inputs (katago-rs_amd/synth.py). A step is
one forward pass of the batch plus the readback of all outputs to the host and a sum over them, as the
reference's bench does (crates/katago-nn-burn/examples/bench.rs:34-41); inputs are already in HBM when timing
starts.

Prints one JSON line. Besides the throughput it carries
- "roofline": the dominant kernel class's algorithmic work per launch over its average launch time, measured
  with HIP events around every kernel launch on the library's stream during a second timed region of the same
  K steps (events need eager launches; the throughput region replays a HIP graph);
- "cpu_baseline": the float32 CPU oracle on bounded samples of the same workload and of b10c128 at batch 8, on one
  thread and on all the host cores this run may use (at most 16), with the host's CPU model and core count, beside
  the reference's published single-thread flex figures (README.md:89, 98 of the reference);
- "roofline.traffic": HBM bytes per launch of the dominant kernel class, from the rocprofv3 FETCH_SIZE and
  WRITE_SIZE passes recorded in profiles/traffic.json (each scaled by the same counter's reading for a device copy
  of known size, `--copy-probe-mb`); null when no measurement for that class and workload is recorded;
- "roofline.rocprof": the same kernel's average duration in the committed rocprofv3 kernel trace of this command
  (profiles/kernel_trace.json, which names the build it was taken on) and the fraction it gives, beside the
  event-timed one;
- "other_workloads": b10c128 float32 at batch 8 (the reference's CPU-runnable config) on the GPU, beside the
  reference's published RX 6800 XT figure.
"""

import argparse
import ctypes
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = {"f16": 2500.0, "bf16": 2500.0, "f32": 157.3}  # MI355X dense MFMA
PEAK_HBM_GBS = 8000.0
# The headline metric's name for the default workload; other workloads are named the same way.
HEADLINE = "evals/s b18c384nbt fp16 batch 32 on 1 MI355X; MFMA util % + HBM GB/s %"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
TRACE_FILE = os.path.join(ROOT, "profiles", "kernel_trace.json")
# The reference's published single-thread flex (burn CPU) throughput, i7-8700K (README.md:89, 98), evals/s.
PUBLISHED_FLEX = {"b10c128 batch 8": 33.0, "b18c384nbt batch 8": 2.5}
# The reference's published ROCm f32 throughput of b10c128 at batch 8 on an RX 6800 XT (README.md:85-86), evals/s.
PUBLISHED_B10C128_F32_B8 = 2617.0


def copy_probe(mb):
    """One device-to-device copy of `mb` MiB (a copy kernel of known size for counter calibration)."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    hip.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    n = mb << 20
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(a), n) == 0 and hip.hipMalloc(ctypes.byref(b), n) == 0
    assert hip.hipMemset(a, 1, n) == 0
    for _ in range(3):
        assert hip.hipMemcpy(b, a, n, 3) == 0  # hipMemcpyDeviceToDevice
    assert hip.hipDeviceSynchronize() == 0
    hip.hipFree(a)
    hip.hipFree(b)
    print(json.dumps({"copy_probe_bytes": n}))


def _recorded(path, kernel, workload):
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    return rec.get(workload, {}).get(kernel)


def recorded_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from the committed counter passes, or None."""
    e = _recorded(TRAFFIC_FILE, kernel, workload)
    return None if e is None else e.get("bytes_per_launch")


def recorded_trace_us(kernel, workload):
    """The average duration (us) of `kernel` on `workload` in the committed rocprofv3 kernel trace, or None."""
    e = _recorded(TRACE_FILE, kernel, workload)
    return None if e is None else e.get("avg_us")


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def time_oracle(oracle, synth, config, rows, threads):
    """evals/s of the float32 CPU oracle on `rows` rows of `config`'s benchmark inputs (one warm-up row first)."""
    arch_fn, _ = synth.CONFIGS[config]
    arch = arch_fn()
    om = oracle.Model(synth.write_model(arch, synth.CONFIG_SEEDS[config]))
    sp, gl, me = synth.make_inputs(rows, 1234, meta=arch.meta_encoder)
    om.forward(sp[:1], gl[:1], None if me is None else me[:1], dtype=np.float32, threads=threads)
    t = time.perf_counter()
    om.forward(sp, gl, me, dtype=np.float32, threads=threads)
    dt = time.perf_counter() - t
    return {"value": rows / dt, "rows": rows, "threads": threads, "seconds": round(dt, 2)}


def time_gpu_workload(kgx, synth, hip, config, precision, batch, steps, warmup):
    """evals/s of `config` at `batch` on the GPU: inputs resident, each step one forward and its readback."""
    arch_fn, _ = synth.CONFIGS[config]
    arch = arch_fn()
    net = kgx.Net(synth.write_model(arch, synth.CONFIG_SEEDS[config]))
    h = kgx.Handle(net, batch, precision, device=0)
    sp, gl, me = synth.make_inputs(batch, 1234, meta=arch.meta_encoder)
    d_bin, d_glob, d_meta, _ = h.device_buffers()
    assert hip.hipMemcpy(d_bin, sp.ctypes.data, sp.nbytes, 1) == 0
    assert hip.hipMemcpy(d_glob, gl.ctypes.data, gl.nbytes, 1) == 0
    if me is not None:
        assert hip.hipMemcpy(d_meta, me.ctypes.data, me.nbytes, 1) == 0
    out = np.empty((batch, net.row_len), np.float32)
    for _ in range(warmup):
        h.run(batch, out)
    h.sync()
    t = time.perf_counter()
    for _ in range(steps):
        h.run(batch, out)
        out.sum(dtype=np.float64)
    dt = time.perf_counter() - t
    h.close()
    return {"value": batch * steps / dt, "unit": "evals/s", "ms_per_step": dt / steps * 1e3, "steps": steps}


def time_featurizer(kgx, synth, hip, net, precision, batch, steps):
    """The device featurizer (kg_featurize) and the whole device path (kg_evaluate_positions: featurizer, forward
    pass, post-processing, one readback of the finished fields) on `batch` seeded 19x19 positions. The featurizer is
    timed with HIP events on the handle's stream around its upload and kernel; the whole path by the wall clock per
    call, as a caller sees it."""
    h = kgx.Handle(net, batch, precision, device=0)
    pos = kgx.make_positions(synth.make_positions(batch, 77))
    sym = np.ascontiguousarray(np.arange(batch) % 8, np.int32)
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    stream = ctypes.c_void_p(h.stream)
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipEventCreate(ctypes.byref(e0)) == 0 and hip.hipEventCreate(ctypes.byref(e1)) == 0
    for _ in range(5):
        h.featurize(pos, sym)
    h.sync()
    reps = max(steps, 20)
    assert hip.hipEventRecord(e0, stream) == 0
    for _ in range(reps):
        h.featurize(pos, sym)
    assert hip.hipEventRecord(e1, stream) == 0
    assert hip.hipEventSynchronize(e1) == 0
    ms = ctypes.c_float()
    assert hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1) == 0
    us = ms.value * 1e3 / reps
    hip.hipEventDestroy(e0)
    hip.hipEventDestroy(e1)
    # 1552 bytes read and 22 * 361 + 19 floats written per position
    bytes_per_batch = batch * (ctypes.sizeof(kgx.Position) + (22 * 361 + 19) * 4)
    # The whole device path, with its ctypes arguments built once (the caller's own marshalling is not timed).
    lib = kgx.lib()
    legal = [np.concatenate([np.ones(361, np.uint8), np.ones(1, np.uint8)]) for _ in range(batch)]
    post = (kgx.PostInput * batch)()
    for i in range(batch):
        post[i].legal = legal[i].ctypes.data
        post[i].white_to_move = int(pos[i].next_player == 2)
        post[i].board_x_size = post[i].board_y_size = 19
        post[i].nn_policy_temperature = 1.0
        post[i].enable_passing_hacks = 0
        post[i].no_result_allowed = 1
    outs = (kgx.NNOutput * batch)()
    owners = [np.zeros(361, np.float32) for _ in range(batch)]
    for i in range(batch):
        outs[i].white_owner_map = owners[i].ctypes.data
    opt = np.zeros(batch, np.float32)
    call = lambda: lib.kg_evaluate_positions(h._h, batch, pos, sym.ctypes.data, opt.ctypes.data, post, outs)
    for _ in range(5):
        assert call() == 0, lib.kg_last_error().decode()
    t = time.perf_counter()
    for _ in range(steps):
        assert call() == 0, lib.kg_last_error().decode()
    dt = time.perf_counter() - t
    h.close()
    return {"positions": batch, "featurize_us_per_batch": us,
            "featurize_note": "kg_featurize: upload of the positions and the kernel, HIP events on the handle's stream",
            "featurize_gbs": bytes_per_batch / (us * 1e-6) / 1e9,
            "featurize_bytes_per_batch": bytes_per_batch,
            "evaluate_positions": {"value": batch * steps / dt, "unit": "evals/s", "ms_per_call": dt / steps * 1e3,
                                   "note": "kg_evaluate_positions: positions to NNEvaluator's fields, featurizer, "
                                           "forward, post-processing and one readback on the device"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="b18c384nbt")
    ap.add_argument("--precision", default="f16", choices=["f16", "bf16", "f32"])
    ap.add_argument("--batch", type=int, default=0, help="override the config's batch size")
    ap.add_argument("--cpu-rows", type=int, default=-1,
                    help="rows in the all-core CPU-baseline sample (-1: the whole batch, 0: skip the CPU baseline)")
    ap.add_argument("--cpu-rows-1t", type=int, default=2, help="rows in the single-thread CPU-baseline sample")
    ap.add_argument("--cpu-threads", type=int, default=0, help="CPU-baseline threads (0: min(16, cores))")
    ap.add_argument("--other-workloads", type=int, default=1, help="also time b10c128 f32 batch 8 (0: skip)")
    ap.add_argument("--handles", type=int, default=2,
                    help="also time this many handles in flight, one thread each (reported as 'pipelined'; 1: skip)")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="only run a device copy of this many MiB (counter calibration) and exit")
    args = ap.parse_args()

    if args.copy_probe_mb:
        copy_probe(args.copy_probe_mb)
        return

    if args.gpus != 1:
        print(json.dumps({"error": "this path runs on one GPU; the forward pass shards by independent batches "
                                   "with no collective, so a multi-GPU figure is N independent copies. Use --gpus 1."}))
        sys.exit(2)

    kgx = importlib.import_module("katago-rs_amd")
    synth = importlib.import_module("katago-rs_amd.synth")

    arch_fn, batch = synth.CONFIGS[args.config]
    if args.batch:
        batch = args.batch
    arch = arch_fn()
    model = synth.write_model(arch, synth.CONFIG_SEEDS[args.config])
    net = kgx.Net(model)
    h = kgx.Handle(net, batch, args.precision, device=0)
    sp, gl, me = synth.make_inputs(batch, 1234, meta=arch.meta_encoder)

    # Inputs resident in HBM: copy them into the handle's device buffers once.
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    d_bin, d_glob, d_meta, _ = h.device_buffers()
    assert hip.hipMemcpy(d_bin, sp.ctypes.data, sp.nbytes, 1) == 0
    assert hip.hipMemcpy(d_glob, gl.ctypes.data, gl.nbytes, 1) == 0
    if me is not None:
        assert hip.hipMemcpy(d_meta, me.ctypes.data, me.nbytes, 1) == 0

    out = np.empty((batch, net.row_len), np.float32)

    def step():
        h.run(batch, out)  # forward + readback into `out` + wait

    # (The checksum of the outputs is host work of this script, not of the forward pass: it is taken from the last
    # step's rows after the timed region, 19 us per batch-32 step on one core.)
    for _ in range(args.warmup):
        step()
    h.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    h.sync()
    dt = time.perf_counter() - t0
    checksum = float(out.sum(dtype=np.float64))
    ms_per_step = dt / args.steps * 1e3
    evals_per_s = batch * args.steps / dt
    if not np.isfinite(checksum):
        raise RuntimeError("non-finite outputs")
    # The reference bench's own method beside the exact K steps: at least 8 iterations and at least 2 s
    # (crates/katago-nn-burn/examples/bench.rs:49-53).
    ns, t0 = 0, time.perf_counter()
    while ns < 8 or time.perf_counter() - t0 < 2.0:
        step()
        ns += 1
    h.sync()
    sdt = time.perf_counter() - t0
    sustained = {"value": batch * ns / sdt, "steps": ns, "seconds": round(sdt, 3),
                 "method": "at least 8 iterations and at least 2 s, as the reference's examples/bench.rs"}

    # Second timed region: the same K steps launched eagerly with HIP events around every kernel.
    h.profile(True)
    h.profile_reset()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    prof_ms_per_step = (time.perf_counter() - t1) / args.steps * 1e3
    prof = h.profile_read()
    h.profile(False)
    total_kernel_ms = sum(v["ms"] for v in prof.values())
    classes = {}
    for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"]):
        n = max(v["launches"], 1)
        avg_ms = v["ms"] / n
        c = {"launches_per_step": v["launches"] / args.steps, "avg_us": avg_ms * 1e3,
             "share": v["ms"] / total_kernel_ms if total_kernel_ms else 0.0}
        # Both roofline fractions of every class (algorithmic flops and bytes per launch over its event time):
        # latency-bound kernels reach neither, and the 1x1 convolutions' bound is the higher one.
        if v["flops"] > 0:
            c["tflops"] = v["flops"] / (v["ms"] * 1e-3) / 1e12
            c["mfma_frac"] = c["tflops"] / PEAK_TFLOPS[args.precision]
        if v["bytes"] > 0:
            c["gbs"] = v["bytes"] / (v["ms"] * 1e-3) / 1e9
            c["hbm_frac"] = c["gbs"] / PEAK_HBM_GBS
        classes[k] = c
    dom = max(prof.items(), key=lambda kv: kv[1]["ms"])
    dname, dv = dom
    per_launch_ms = dv["ms"] / max(dv["launches"], 1)
    if dv["flops"] > 0:
        achieved = dv["flops"] / max(dv["launches"], 1) / (per_launch_ms * 1e-3) / 1e12
        peak = PEAK_TFLOPS[args.precision]
        roof = {"bound": "mfma", "kernel": dname, "achieved": achieved, "peak": peak, "unit": "TFLOP/s",
                "frac": achieved / peak, "traffic": None,
                "work_per_launch": dv["flops"] / max(dv["launches"], 1), "avg_launch_us": per_launch_ms * 1e3}
    else:
        achieved = dv["bytes"] / max(dv["launches"], 1) / (per_launch_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": dname, "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_HBM_GBS, "traffic": None,
                "work_per_launch": dv["bytes"] / max(dv["launches"], 1), "avg_launch_us": per_launch_ms * 1e3}
    # Several handles in flight (one engine thread per handle, as the reference's serve tasks, docs/M9-report.md):
    # each step is still one batch's forward + readback, on its handle's own stream; the handles' kernels fill
    # each other's gaps. Reported beside the single-forward value, not as it.
    pipelined = None
    if args.handles > 1:
        import threading
        hs = [h] + [kgx.Handle(net, batch, args.precision, device=0) for _ in range(args.handles - 1)]
        for hh in hs[1:]:
            db, dg, dm, _ = hh.device_buffers()
            assert hip.hipMemcpy(db, sp.ctypes.data, sp.nbytes, 1) == 0
            assert hip.hipMemcpy(dg, gl.ctypes.data, gl.nbytes, 1) == 0
            if me is not None:
                assert hip.hipMemcpy(dm, me.ctypes.data, me.nbytes, 1) == 0

        def loop(hh, k):
            o = np.empty((batch, net.row_len), np.float32)
            for _ in range(k):
                hh.run(batch, o)

        for hh in hs:
            loop(hh, args.warmup)
        ths = [threading.Thread(target=loop, args=(hh, args.steps)) for hh in hs]
        t2 = time.perf_counter()
        for t in ths:
            t.start()
        for t in ths:
            t.join()
        pdt = time.perf_counter() - t2
        pipelined = {"handles": args.handles, "value": args.handles * batch * args.steps / pdt, "unit": "evals/s",
                     "steps_per_handle": args.steps}
        for hh in hs[1:]:
            hh.close()
    h.close()

    workload = f"{args.config} {args.precision} batch {batch}"
    roof["traffic"] = recorded_traffic(dname, workload)

    rp_us = recorded_trace_us(dname, workload)
    if rp_us:
        roof["rocprof"] = {"avg_launch_us": rp_us, "achieved": roof["work_per_launch"] / (rp_us * 1e-6) /
                           (1e12 if roof["unit"] == "TFLOP/s" else 1e9)}
        roof["rocprof"]["frac"] = roof["rocprof"]["achieved"] / roof["peak"]
        roof["rocprof"]["source"] = ("profiles/kernel_trace.json: rocprofv3 --kernel-trace --stats of this command "
                                     "on the build recorded there (not the build that ran here)")

    featurizer = time_featurizer(kgx, synth, hip, net, args.precision, batch, args.steps) if (
        net.num_input_channels == 22 and net.num_global == 19 and net.num_meta == 0) else None

    other = None
    if args.other_workloads and (args.config, args.precision, batch) == ("b18c384nbt", "f16", 32):
        r = time_gpu_workload(kgx, synth, hip, "b10c128", "f32", 8, max(args.steps, 100), args.warmup)
        r["published_rx6800xt_rocm_f32"] = PUBLISHED_B10C128_F32_B8
        other = {"b10c128 f32 batch 8": r}

    cpu = None
    if args.cpu_rows < 0:
        args.cpu_rows = batch
    if args.cpu_rows > 0:
        import oracle
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        n = min(args.cpu_rows, batch)
        allc = time_oracle(oracle, synth, args.config, n, threads)
        one = time_oracle(oracle, synth, args.config, max(1, args.cpu_rows_1t), 1)
        cpu = {"value": allc["value"], "unit": "evals/s", "cores": threads, "kind": "port",
               "sample": f"{n} rows of the same workload through the float32 CPU oracle (direct convolution, "
                         f"plain loops) on {threads} threads, {allc['seconds']} s",
               "single_thread": one, "nproc": os.cpu_count(), "cpu_model": cpu_model(),
               "published_flex_1_thread_i7_8700k": PUBLISHED_FLEX}
        if args.config == "b18c384nbt":
            cpu["b10c128 batch 8"] = {"all_cores": time_oracle(oracle, synth, "b10c128", 8, threads),
                                      "single_thread": time_oracle(oracle, synth, "b10c128", 8, 1)}
            cpu["note"] = ("The oracle is a plain-loop restatement: per core it runs "
                           f"{PUBLISHED_FLEX['b18c384nbt batch 8'] / max(one['value'], 1e-9):.1f}x slower than "
                           "the reference's published flex figure for b18c384nbt (different CPU, batch 8).")

    res = {
        "metric": HEADLINE if (args.config, args.precision, batch) == ("b18c384nbt", "f16", 32) else
                  f"evals/s {args.config} {'fp16' if args.precision == 'f16' else args.precision} batch {batch} "
                  "on 1 MI355X; MFMA util % + HBM GB/s %",
        "value": evals_per_s,
        "unit": "evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.precision,
        "data": "synthetic: seeded random-init weights of the named architecture and seeded Bernoulli(0.3) inputs",
        "config": {"workload": f"{args.config} forward pass, batch {batch}, 19x19, {args.precision} GEMM operands, "
                               "float accumulate, one readback per batch", "batch": batch,
                   "network": args.config},
        "roofline": roof,
        "cpu_baseline": cpu,
        "kernels": classes,
        "profiled_ms_per_step": prof_ms_per_step,
        "checksum": checksum,
        "pipelined": pipelined,
        "other_workloads": other,
        "sustained": sustained,
        "featurizer": featurizer,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
