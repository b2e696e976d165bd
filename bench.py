"""MoE-layer throughput benchmark on one MI355X.

A step is one pass of the hot path over one batch: one MoE feed-forward block
(router, top-k, dispatch, routed experts, shared expert, combine) over T
tokens, or for config 4 the whole 40-layer stack (RMSNorm + MoE + residual per
layer).  Inputs and all weights are resident in HBM before timing; the timed
steps replay a HIP graph.  Layer-mode configs rotate over several
independently seeded layers and a bank of seeded inputs, so the routed
experts of a step are cold in the 256 MB last-level cache; the warm-up runs on
layers and inputs of its own, disjoint from the timed ones, whatever --steps
is.

Default (no --config): BASELINE's metric is quoted on two workloads, B=1
decode and B=512 prefill; the line is config 0 (B=1 decode) and carries
config 2 (T=512 prefill, balanced) as "secondary", both timed for --steps
steps, and config 4p (the 40-layer stack over a 2048-token prefill, the
MFMA-bound workload) as "prefill_stack" at its own step count, each with its
own roofline and CPU baseline.  --config C runs one config.

Per config the line holds the roofline of the dominant kernel: algorithmic
bytes (or flops) per launch over that kernel's average duration, measured with
HIP events that its launches record themselves (start when the kernel begins,
stop when it ends) while the timed steps run again back to back on the
context stream (profiles/ holds the rocprofv3 kernel-trace figures of the
same command); the C oracle on this host's cores as the CPU baseline (one thread,
and all cores with OpenMP); and per-stage kernel times.
"""
import argparse
import ctypes as C
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
Q4K, Q6K = 12, 14

# name, tokens/step, mode, timed layers (layer mode) or stack depth, spec,
# input bank, default steps
CONFIGS = {
    "0": dict(T=1, name="moe_decode_b1", mode="layer", layers=8, spec={}, xbank=64, steps=2000),
    "1": dict(T=8, name="moe_decode_b8", mode="layer", layers=8, spec={}, xbank=64, steps=2000),
    "2": dict(T=512, name="moe_prefill_512_balanced", mode="layer", layers=4, spec={}, xbank=4,
              steps=200),
    "3": dict(T=512, name="moe_prefill_512_zipf_q6k", mode="layer", layers=4,
              spec=dict(down=Q6K, zipf=True), xbank=4, steps=200),
    # the layout of common Q4_K_M MoE files: Q5_K routed down, Q8_0 shared
    # expert (not a BASELINE config; a parity-tested variant)
    "2r": dict(T=512, name="moe_prefill_512_q5k_down_q8_shared", mode="layer", layers=4,
               spec=dict(down=13, shared=8), xbank=4, steps=200),
    # one layer over a 2048-token prefill, its routing fixed by the inputs
    # (not a BASELINE config: the layer of config 4p without the stack, for
    # kernel studies whose outputs feed nothing)
    "p2048": dict(T=2048, name="moe_prefill_2048_layer", mode="layer", layers=4, spec={}, xbank=2, steps=40),
    "4d": dict(T=1, name="moe_stack40_decode_b1", mode="stack", layers=40,
               spec=dict(q6k_every=4, centered=True), xbank=16, steps=100),
    "4p": dict(T=2048, name="moe_stack40_prefill_2048", mode="stack", layers=40,
               spec=dict(q6k_every=4, centered=True), xbank=2, steps=4),
}
WARM_LAYERS = 2  # layer mode: extra layers used only by the warm-up


def q4k_bytes(rows, cols):
    return rows * (cols // 256) * 144


def q6k_bytes(rows, cols):
    return rows * (cols // 256) * 210


def mat_bytes(ggml_type, rows, cols):
    """Bytes of a [rows x cols] matrix in a ggml block format (Q4_K, Q5_K, Q6_K, Q8_0)."""
    per = {12: (256, 144), 13: (256, 176), 14: (256, 210), 8: (32, 34)}[ggml_type]
    return rows * (cols // per[0]) * per[1]


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run_config(key, steps, warmup, path, cpu_seconds, no_cpu, graph=True):
    import orome_amd
    from orome_amd import _lib
    from orome_amd._lib import check, lib
    from orome_amd.moe import DeviceBuffer

    cf = CONFIGS[key]
    T, L, NX = cf["T"], cf["layers"], cf["xbank"]
    steps = steps or cf["steps"]
    warmup = warmup if warmup is not None else max(1, steps // 10)
    stack = cf["mode"] == "stack"
    H, E, K, M, S = 2048, 256, 8, 512, 512
    LW = 0 if stack else WARM_LAYERS
    spec = orome_amd.make_spec(layers=L + LW, H=H, E=E, K=K, M=M, S=S, seed=1234, **cf["spec"])
    log("config %s (%s): %d timed + %d warm-up synthetic layers, T=%d" % (key, cf["name"], L, LW, T))
    img = orome_amd.synth_gguf(spec)
    # the library's choice under "auto": GEMV kernels up to 2 tokens, the
    # small-batch routing with the small-tile grouped GEMMs for 3..16, the
    # large-batch routing and grouped GEMMs above
    kpath = path if path != "auto" else ("gemv" if T <= 2 else "small_batch_gemm" if T <= 16 else "mfma")
    gm = orome_amd.MoEModel(image=img, max_tokens=max(T, 16), pack=kpath != "gemv")
    ctx = gm.ctx
    if path != "auto":
        ctx.set_path(_lib.OROME_PATH_MFMA if kpath == "mfma" else _lib.OROME_PATH_GEMV)
    # timed inputs: bank 0..NX-1; warm-up inputs: a bank of their own
    xs_h = [orome_amd.synth_normal(77, i, T * H).reshape(T, H) for i in range(NX)]
    hs_h = [orome_amd.synth_normal(78, i, T * H).reshape(T, H) for i in range(NX)]
    wx_h = [orome_amd.synth_normal(79, i, T * H).reshape(T, H) for i in range(2)]
    xs = [DeviceBuffer.from_array(ctx, v) for v in xs_h]
    hs = [DeviceBuffer.from_array(ctx, v) for v in hs_h]
    wx = [DeviceBuffer.from_array(ctx, v) for v in wx_h]
    outs = [DeviceBuffer(ctx, T * H * 4) for _ in range(2)]

    def step(i):
        if stack:  # h = x_i, then 40 x (h += MoE_l(RMSNorm(h))) in place
            gm.stack_forward(xs[i % NX], T)
        else:
            gm.forward(i % L, xs[i % NX], hs[i % NX], outs[i % 2], T)

    def warm_step(i):
        if stack:
            gm.stack_forward(wx[i % 2], T)
        else:  # warm-up layers L .. L+LW-1 with the warm-up inputs
            gm.forward(L + i % LW, wx[i % 2], wx[(i + 1) % 2], outs[i % 2], T)

    def restore():
        if stack:  # the stack works in place: pristine inputs between runs
            for b, v in zip(xs, xs_h):
                b.upload(v)
            for b, v in zip(wx, wx_h):
                b.upload(v)

    # touched experts per step (weights are counted once per touched expert)
    G = min(steps, 200 if not stack else max(1, min(steps, 10)))
    touched = []
    for i in range(min(G, 64)):
        if stack:
            gm.layer_forward(L - 1, xs[i % NX], T)
        else:
            gm.forward(i % L, xs[i % NX], hs[i % NX], outs[0], T)
        off = gm.debug_outputs(T)["offsets"].astype(np.int64)
        touched.append(int(np.count_nonzero(np.diff(off))))
    restore()
    u_mean = float(np.mean(touched))

    def capture(fn, n):
        check(lib.orome_hip_capture_begin(ctx.handle), "capture")
        for i in range(n):
            fn(i)
        ex = C.c_void_p()
        check(lib.orome_hip_capture_end(ctx.handle, C.byref(ex)), "capture_end")
        return ex

    rem = steps % G
    reps = steps // G
    nwarm = max(1, min(warmup, G))
    if graph:
        g_main = capture(step, G)
        g_rem = capture(step, rem) if rem else None
        g_warm = capture(warm_step, nwarm)
    else:
        g_main = g_rem = g_warm = None

    def warm():
        if g_warm:
            check(lib.orome_hip_graph_launch(ctx.handle, g_warm))
        else:
            for i in range(nwarm):
                warm_step(i)

    for _ in range(max(1, math.ceil(warmup / G))):
        warm()
    ctx.sync()
    # zero-length k_delay dispatches mark the regions for a kernel trace:
    # the 1st and 2nd bracket the timed steps, the 3rd (the stage timing's
    # spin) and 4th the per-stage event pass
    mark = lambda: check(lib.orome_hip_stream_delay(ctx.handle, 0))
    mark()
    if graph:
        t0 = time.perf_counter()
        for _ in range(reps):
            check(lib.orome_hip_graph_launch(ctx.handle, g_main))
        if g_rem:
            check(lib.orome_hip_graph_launch(ctx.handle, g_rem))
        ctx.sync()
        elapsed = time.perf_counter() - t0
    else:
        # --no-graph: the timed steps launched eagerly, so the wall clock
        # holds the host's launch cost too (a profiling mode, not the figure)
        t0 = time.perf_counter()
        for i in range(steps):
            step(i)
        ctx.sync()
        elapsed = time.perf_counter() - t0
    mark()
    restore()

    # per-kernel durations: the timed steps launched again, eagerly, on the
    # context stream, each stage's kernels recording its event pair
    # (orome_hip_stage_timing), all queued behind a GPU-side delay so that
    # they run back to back as in the graph; after a warm-up replay
    n_prof = min(steps, G)
    warm()
    check(lib.orome_hip_stage_timing(ctx.handle, n_prof * (L if stack else 1)))
    check(lib.orome_hip_stream_delay(ctx.handle, 200000))
    for i in range(n_prof):
        step(i)
    tot = (C.c_float * 8)()
    cnt = (C.c_int * 8)()
    mark()
    check(lib.orome_hip_stage_times(ctx.handle, tot, cnt, 8))
    check(lib.orome_hip_stage_timing(ctx.handle, 0))
    stage_us = {_lib.STAGES[i]: (round(tot[i] / cnt[i] * 1000.0, 3) if cnt[i] else None) for i in range(8)}
    restore()

    # in-kernel view of the same launches: every block of the gate/up kernels
    # stamps its start and end (s_memrealtime); first start to last end
    KTB = 16384
    ktbuf = DeviceBuffer(ctx, KTB * 2 * 8)
    zeros = np.zeros(KTB * 2, np.uint64)
    check(lib.orome_hip_kernel_timing(ctx.handle, ktbuf.ptr, KTB), "kernel_timing")
    spans = []
    for i in range(40):
        ktbuf.upload(zeros)
        if stack:
            gm.layer_forward(i % L, xs[i % NX], T)
        else:
            gm.forward(i % L, xs[i % NX], hs[i % NX], outs[i % 2], T)
        ctx.sync()
        v = ktbuf.download(np.uint64, (KTB, 2)).astype(np.int64)
        ok = (v[:, 0] > 0) & (v[:, 1] > 0)
        spans.append((v[ok, 1].max() - v[ok, 0].min()) * 0.01)  # 100 MHz ticks -> us
    check(lib.orome_hip_kernel_timing(ctx.handle, None, 0), "kernel_timing")
    ktbuf.free()
    restore()

    # algorithmic work per gate/up launch and per MoE layer
    nl = L if stack else 1
    n_q6 = sum(1 for l in range(L) if cf["spec"].get("q6k_every") and l % 4 == 3) if stack else 0
    down_e = mat_bytes(cf["spec"].get("down", Q4K), H, M)
    sh_t = cf["spec"].get("shared", Q4K)
    rows = T * K + T  # routed pairs plus shared-expert rows
    gu_bytes = (u_mean * 2 * q4k_bytes(M, H) + 2 * mat_bytes(sh_t, S, H) + T * H * (4 if kpath == "gemv" else 2)
                + rows * M * 2)
    gu_flops = 2.0 * 2 * rows * M * H
    layer_bytes = (u_mean * (2 * q4k_bytes(M, H) + down_e) + 2 * mat_bytes(sh_t, S, H) + mat_bytes(sh_t, H, S)
                   + E * H * 4 + H * 4 + T * H * 4 * 3)
    if stack:
        layer_bytes += (q6k_bytes(H, M) - q4k_bytes(H, M)) * u_mean * n_q6 / L
    step_bytes = layer_bytes * nl
    step_flops = 2.0 * (rows * M * H * 3 + T * (E + 1) * H) * nl
    gu_us = stage_us["gate_up"]
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    gu_tflops = gu_flops / (gu_us * 1e-6) / 1e12
    # up to T K = 32 E every expert is in 32-row tiles (one list); above, the
    # 32-row and 80-row tile lists
    kname = {"gemv": "gemv_gate_up", "small_batch_gemm": "gemm_gate_up (16-row tiles)",
             "mfma": ("gemm_gate_up (32-row tile list)" if T * K <= 32 * E
                      else "gemm_gate_up (32-row + 80-row tile lists)")}[kpath]
    if T >= 2048:
        roof = {"bound": "mfma", "kernel": kname, "achieved": round(gu_tflops, 2),
                "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(gu_tflops / MFMA_F16_PEAK_TFLOPS, 4)}
    else:
        roof = {"bound": "hbm", "kernel": kname, "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4)}
    # the committed profile of this workload: HBM traffic per launch (two
    # rocprofv3 --pmc passes) and the kernel-trace average of the gate/up
    # stage over the timed steps (a kernel trace cut at the region marks)
    traffic, rp = None, {}
    tf = os.path.join(ROOT, "profiles", "traffic_%s.json" % cf["name"])
    if os.path.exists(tf):
        rp = json.load(open(tf))
        traffic = rp.get("gate_up_hbm_bytes_per_launch")
    serial = kpath == "mfma" and T * K > 32 * E
    roof.update({"traffic": traffic, "algorithmic_bytes_per_launch": int(gu_bytes),
                 "algorithmic_flops_per_launch": gu_flops, "avg_launch_us": gu_us,
                 "timing": "HIP events recorded by the gate/up launches themselves (hipExtLaunchKernel "
                           "start/stop, on the launch's stream), the timed steps relaunched back to back "
                           "(%d launches)%s" % (n_prof * nl,
                                                "; under stage timing the two tile lists run one after the "
                                                "other on one stream, where the timed steps overlap them on two"
                                                if serial else ""),
                 "in_kernel_us": round(float(np.mean(spans)), 3),
                 "gbs": round(gu_gbs, 1), "tflops": round(gu_tflops, 2)})
    if rp.get("rocprof_gate_up_avg_us"):
        ra = rp["rocprof_gate_up_avg_us"]
        roof["rocprof"] = {"avg_launch_us": ra, "source": rp.get("rocprof_source"),
                           "frac": round((gu_flops / (ra * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS) if T >= 2048
                                         else (gu_bytes / (ra * 1e-6) / 1e9 / HBM_PEAK_GBS), 4),
                           "events_over_rocprof": round(gu_us / ra, 4)}
    fmts = {12: "q4_k", 13: "q5_k", 14: "q6_k", 8: "q8_0"}
    dn = fmts[cf["spec"].get("down", Q4K)] + ("/q6_k (every 4th layer)" if stack else "")
    dtype = ("routed gate/up q4_k, routed down %s, shared %s weights; fp16 activations, fp32 accumulate"
             % (dn, fmts[sh_t]))

    cpu = None if no_cpu else cpu_baseline(img, xs_h, hs_h, T, L, NX, nl, stack, cpu_seconds)

    value = T * steps / elapsed
    out = {
        "metric": "MoE-layer tokens/s" if not stack else "MoE 40-layer stack tokens/s",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(elapsed / steps * 1000, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic seeded GGUF per BASELINE config %s (%d timed layers, %d input batches; warm-up on "
                "%d layers and inputs of its own)" % (key, L, NX, LW),
        "config": {"workload": cf["name"], "baseline_config": key, "tokens_per_step": T,
                   "kernel_path": kpath, "launch": "hip graph" if graph else "eager (--no-graph)",
                   "layers_per_step": nl, "hidden": H, "experts": E, "top_k": K,
                   "expert_intermediate": M, "shared_intermediate": S, "parallelism": "single GPU"},
        "roofline": roof,
        "step": {"algorithmic_bytes": int(step_bytes), "touched_experts_per_layer": u_mean,
                 "gbs": round(step_bytes * steps / elapsed / 1e9, 1),
                 "hbm_frac": round(step_bytes * steps / elapsed / 1e9 / HBM_PEAK_GBS, 4),
                 "tflops": round(step_flops * steps / elapsed / 1e12, 2),
                 "mfma_frac": round(step_flops * steps / elapsed / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                 "us_per_layer": round(elapsed / steps / nl * 1e6, 3)},
        "stage_us": stage_us,
        "cpu_baseline": cpu,
    }
    for g in (g_main, g_rem, g_warm):
        if g:
            lib.orome_hip_graph_destroy(g)
    gm.close()
    return out


def cpu_baseline(img, xs_h, hs_h, T, L, NX, nl, stack, seconds):
    """The C oracle (scalar, -O2) on this host: one thread for `seconds`, then
    OpenMP over all the threads OMP_NUM_THREADS allows for half as long, on
    the first (up to) 64 tokens of each input batch.  Rates are tokens/s of a
    full step (nl layers)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    om = O.OracleModel(img)
    tsub = min(T, 64)

    def timed(omp, secs):
        n = 0
        c0 = time.perf_counter()
        while time.perf_counter() - c0 < secs:
            xi = xs_h[n % NX][:tsub]
            if stack:
                om.layer_forward(n % L, xi.copy(), omp=omp)
            else:
                om.forward(n % L, xi, hs_h[n % NX][:tsub], omp=omp)
            n += 1
        ct = time.perf_counter() - c0
        return n, ct, n * tsub / ct / nl

    n1, t1, r1 = timed(False, seconds)
    threads = int(O.lib(True).orc_num_threads())
    nm, tm, rm = timed(True, seconds / 2)
    sample = "first %d token(s) of each batch" % tsub if tsub < T else "full batch"
    scaled = "; scaled to the %d-layer step" % nl if nl > 1 else ""
    return {"value": round(r1, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": "%d single-layer passes of %d token(s) (%s), scalar C oracle (-O2), 1 thread, %.1f s%s"
                      % (n1, tsub, sample, t1, scaled),
            "all_cores": {"value": round(rm, 4), "unit": "tokens/s", "cores": threads,
                          "sample": "%d passes as above, OpenMP over output rows and tokens, %d threads, %.1f s"
                                    % (nm, threads, tm)},
            "host": {"nproc": os.cpu_count(), "cpu_model": cpu_model()}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", default=None, choices=sorted(CONFIGS),
                    help="one config; default: config 0 with config 2 as the secondary workload")
    ap.add_argument("--path", default="auto", choices=["auto", "gemv", "mfma"],
                    help="kernel path (auto: GEMV up to 2 tokens, small-batch routing with the small-tile "
                         "grouped GEMMs for 3..16, large-batch routing and grouped GEMMs above)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the timed steps eagerly instead of replaying a HIP graph (a profiling mode)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="run only a plain device-to-device copy of MIB MiB (5 times), the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the MoE path is single-GPU; "
              "expert-parallel sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        import torch
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": n, "launches": 5}))
        return

    kw = dict(graph=not args.no_graph)
    if args.config is not None:
        out = run_config(args.config, args.steps, args.warmup, args.path, args.cpu_seconds, args.no_cpu, **kw)
    else:
        out = run_config("0", args.steps, args.warmup, args.path, args.cpu_seconds, args.no_cpu, **kw)
        keys = ("metric", "value", "unit", "steps", "warmup", "ms_per_step", "dtype", "config", "roofline", "step",
                "stage_us", "cpu_baseline", "data")
        sec = run_config("2", args.steps, args.warmup, args.path, args.cpu_seconds / 2, args.no_cpu, **kw)
        out["secondary"] = {k: sec[k] for k in keys}
        # the 40-layer T=2048 prefill stack: the MFMA-bound workload (its own
        # default step count; --steps applies to the two above)
        pre = run_config("4p", None, None, args.path, args.cpu_seconds / 2, args.no_cpu, **kw)
        out["prefill_stack"] = {k: pre[k] for k in keys}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
