"""MoE-layer throughput benchmark on one MI355X.

A step is one pass of the hot path over one batch: one MoE feed-forward block
(router, top-k, dispatch, routed experts, shared expert, combine) over T
tokens, or for config 4 the whole 40-layer stack (RMSNorm + MoE + residual per
layer).  Inputs and all weights are resident in HBM before timing; the timed
steps replay a HIP graph.  Layer-mode configs rotate over several
independently seeded layers and a bank of seeded inputs, so the routed
experts of a step are mostly cold in the 256 MB last-level cache.

Default (no flags): config 0, B=1 decode, the headline of BASELINE.json.
Prints one JSON line; extra fields hold the roofline of the dominant kernel
(per-launch HIP event timing inside a replay of the same graph), the C
oracle on this host as CPU baseline, and per-stage kernel times.
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

# name, tokens/step, mode, rotating layers (layer mode) or stack depth, spec
CONFIGS = {
    "0": dict(T=1, name="moe_decode_b1", mode="layer", layers=8, spec={}, xbank=64, steps=2000),
    "1": dict(T=8, name="moe_decode_b8", mode="layer", layers=8, spec={}, xbank=64, steps=2000),
    "2": dict(T=512, name="moe_prefill_512_balanced", mode="layer", layers=4, spec={}, xbank=4,
              steps=200),
    "3": dict(T=512, name="moe_prefill_512_zipf_q6k", mode="layer", layers=4,
              spec=dict(down=Q6K, zipf=True), xbank=4, steps=200),
    "4d": dict(T=1, name="moe_stack40_decode_b1", mode="stack", layers=40,
               spec=dict(q6k_every=4, centered=True), xbank=16, steps=100),
    "4p": dict(T=2048, name="moe_stack40_prefill_2048", mode="stack", layers=40,
               spec=dict(q6k_every=4, centered=True), xbank=2, steps=4),
}


def q4k_bytes(rows, cols):
    return rows * (cols // 256) * 144


def q6k_bytes(rows, cols):
    return rows * (cols // 256) * 210


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", default="0", choices=sorted(CONFIGS))
    ap.add_argument("--path", default="auto", choices=["auto", "gemv", "mfma"],
                    help="kernel path (auto: GEMV up to 2 tokens, small-batch routing with the small-tile "
                         "grouped GEMMs for 3..16, large-batch routing and grouped GEMMs above)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
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

    import orome_amd
    from orome_amd import _lib
    from orome_amd._lib import check, lib
    from orome_amd.moe import DeviceBuffer

    cf = CONFIGS[args.config]
    T, L, NX = cf["T"], cf["layers"], cf["xbank"]
    steps = args.steps or cf["steps"]
    warmup = args.warmup if args.warmup is not None else max(1, steps // 10)
    H, E, K, M, S = 2048, 256, 8, 512, 512
    spec = orome_amd.make_spec(layers=L, H=H, E=E, K=K, M=M, S=S, seed=1234, **cf["spec"])
    print("[bench] config %s (%s): %d synthetic layers, T=%d" % (args.config, cf["name"], L, T),
          file=sys.stderr, flush=True)
    img = orome_amd.synth_gguf(spec)
    # the library's choice under "auto": GEMV kernels up to 2 tokens, the
    # small-batch routing with the small-tile grouped GEMMs for 3..16, the
    # large-batch routing and grouped GEMMs above
    kpath = args.path if args.path != "auto" else ("gemv" if T <= 2 else "small_batch_gemm" if T <= 16 else "mfma")
    gm = orome_amd.MoEModel(image=img, max_tokens=max(T, 16), pack=kpath != "gemv")
    ctx = gm.ctx
    if args.path != "auto":
        ctx.set_path(_lib.OROME_PATH_MFMA if kpath == "mfma" else _lib.OROME_PATH_GEMV)
    stack = cf["mode"] == "stack"
    xs_h = [orome_amd.synth_normal(77, i, T * H).reshape(T, H) for i in range(NX)]
    hs_h = [orome_amd.synth_normal(78, i, T * H).reshape(T, H) for i in range(NX)]
    xs = [DeviceBuffer.from_array(ctx, v) for v in xs_h]
    hs = [DeviceBuffer.from_array(ctx, v) for v in hs_h]
    outs = [DeviceBuffer(ctx, T * H * 4) for _ in range(2)]

    def step(i):
        if stack:  # h = x_i, then 40 x (h += MoE_l(RMSNorm(h))) in place
            gm.stack_forward(xs[i % NX], T)
        else:
            gm.forward(i % L, xs[i % NX], hs[i % NX], outs[i % 2], T)

    if stack:
        # the stack works in place: keep pristine copies to restore between runs
        def restore():
            for b, v in zip(xs, xs_h):
                b.upload(v)
    else:
        def restore():
            pass

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

    def capture(n):
        check(lib.orome_hip_capture_begin(ctx.handle), "capture")
        for i in range(n):
            step(i)
        ex = C.c_void_p()
        check(lib.orome_hip_capture_end(ctx.handle, C.byref(ex)), "capture_end")
        return ex

    g_main = capture(G)
    rem = steps % G
    g_rem = capture(rem) if rem else None
    reps = steps // G
    for _ in range(max(1, math.ceil(warmup / G))):
        check(lib.orome_hip_graph_launch(ctx.handle, g_main))
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        check(lib.orome_hip_graph_launch(ctx.handle, g_main))
    if g_rem:
        check(lib.orome_hip_graph_launch(ctx.handle, g_rem))
    ctx.sync()
    elapsed = time.perf_counter() - t0

    # per-kernel durations: the same steps launched eagerly with HIP event
    # pairs around every launch, queued behind a GPU delay so the kernels run
    # back to back (no host launch gaps inside the brackets)
    n_prof = min(steps, 400 if not stack else 8)
    check(lib.orome_hip_stage_timing(ctx.handle, n_prof * (L if stack else 1)))
    check(lib.orome_hip_stream_delay(ctx.handle, 400000))
    for i in range(n_prof):
        step(i)
    tot = (C.c_float * 8)()
    cnt = (C.c_int * 8)()
    check(lib.orome_hip_stage_times(ctx.handle, tot, cnt, 8))
    check(lib.orome_hip_stage_timing(ctx.handle, 0))
    stage_us = {_lib.STAGES[i]: (round(tot[i] / cnt[i] * 1000.0, 3) if cnt[i] else None)
                for i in range(8)}
    restore()

    # gate/up launch durations as a kernel trace reports them: every block of
    # the gate/up kernels stamps its start and end (orome_hip_kernel_timing);
    # a launch lasts from its first block's start to its last block's end
    # (the big- and small-tile launches of the MFMA path together)
    KTB = 16384
    ktbuf = DeviceBuffer(ctx, KTB * 2 * 8)
    zeros = np.zeros(KTB * 2, np.uint64)
    check(lib.orome_hip_kernel_timing(ctx.handle, ktbuf.ptr, KTB), "kernel_timing")
    spans, spans_big, spans_small = [], [], []
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
        for part, lst in ((v[:KTB // 2], spans_big), (v[KTB // 2:], spans_small)):
            okp = (part[:, 0] > 0) & (part[:, 1] > 0)
            if okp.any():
                lst.append((part[okp, 1].max() - part[okp, 0].min()) * 0.01)
    check(lib.orome_hip_kernel_timing(ctx.handle, None, 0), "kernel_timing")
    ktbuf.free()
    restore()

    # algorithmic work per gate/up launch and per MoE layer
    nl = L if stack else 1
    n_q6 = sum(1 for l in range(L) if cf["spec"].get("q6k_every") and l % 4 == 3) if stack else 0
    down_e = q6k_bytes(H, M) if cf["spec"].get("down") == Q6K else q4k_bytes(H, M)
    rows = T * K + T  # routed pairs plus shared-expert rows
    gu_bytes = (u_mean + 1) * 2 * q4k_bytes(M, H) + T * H * (4 if kpath == "gemv" else 2) + rows * M * 2
    gu_flops = 2.0 * 2 * rows * M * H
    layer_bytes = (u_mean * (2 * q4k_bytes(M, H) + down_e) + 3 * q4k_bytes(S, H) + E * H * 4 + H * 4
                   + T * H * 4 * 3)
    if stack:
        layer_bytes += (q6k_bytes(H, M) - q4k_bytes(H, M)) * u_mean * n_q6 / L
    step_bytes = layer_bytes * nl
    step_flops = 2.0 * (rows * M * H * 3 + T * (E + 1) * H) * nl
    gu_us = float(np.mean(spans))
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9
    gu_tflops = gu_flops / (gu_us * 1e-6) / 1e12
    mfma_bound = T >= 2048
    if mfma_bound:
        roof = {"bound": "mfma", "kernel": "gemm_gate_up", "achieved": round(gu_tflops, 2),
                "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(gu_tflops / MFMA_F16_PEAK_TFLOPS, 4)}
    else:
        roof = {"bound": "hbm", "kernel": "gemv_gate_up" if kpath == "gemv" else "gemm_gate_up",
                "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gu_gbs / HBM_PEAK_GBS, 4)}
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic_%s.json" % cf["name"])
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get("gate_up_hbm_bytes_per_launch")
    roof.update({"traffic": traffic, "algorithmic_bytes_per_launch": int(gu_bytes),
                 "algorithmic_flops_per_launch": gu_flops, "avg_launch_us": round(gu_us, 3),
                 "timing": "per-block s_memrealtime stamps of 40 launches (first start to last end)",
                 "event_us": stage_us["gate_up"],
                 "big_tile_us": round(float(np.mean(spans_big)), 3) if spans_big else None,
                 "small_tile_us": round(float(np.mean(spans_small)), 3) if spans_small and T > 8 else None,
                 "gbs": round(gu_gbs, 1), "tflops": round(gu_tflops, 2)})

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        om = O.OracleModel(img)
        tsub = min(T, 64)
        n = 0
        c0 = time.perf_counter()
        while time.perf_counter() - c0 < args.cpu_seconds:
            xi = xs_h[n % NX][:tsub]
            if stack:
                om.layer_forward(n % L, xi.copy(), omp=False)
            else:
                om.forward(n % L, xi, hs_h[n % NX][:tsub], omp=False)
            n += 1
        ct = time.perf_counter() - c0
        rate = n * tsub / ct / nl  # tokens/s for a full step (nl layers)
        cpu = {"value": round(rate, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": "%d single-layer passes of %d token(s) (%s), scalar C oracle, 1 thread, %.1f s%s"
                         % (n, tsub, "first %d of each batch" % tsub if tsub < T else "full batch",
                            ct, "; scaled to the %d-layer step" % nl if nl > 1 else "")}

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
        "dtype": "q4_k/q6_k weights, fp16 activations, fp32 accumulate",
        "data": "synthetic seeded GGUF per BASELINE config %s (%d layers, %d input batches)"
                % (args.config, L, NX),
        "config": {"workload": cf["name"], "baseline_config": args.config, "tokens_per_step": T,
                   "kernel_path": kpath,
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
    print(json.dumps(out), flush=True)
    for g in (g_main, g_rem):
        if g:
            lib.orome_hip_graph_destroy(g)


if __name__ == "__main__":
    main()
