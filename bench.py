"""MoE-layer throughput benchmark (one MI355X).

A step is one MoE feed-forward block (router, top-k, dispatch, routed experts,
shared expert, combine) over one batch of T tokens, all on the GPU through
the C ABI.  The timed steps replay a HIP graph; inputs are resident in HBM
before timing starts.  Weights rotate over several independently seeded
layers and inputs over a bank of seeded vectors, so routed experts are
mostly cold in the 256 MB last-level cache (a single layer is 457 MB of
expert weights, and each step touches a different 8-expert subset).

Prints one JSON line (driver contract).  Extra fields: roofline (dominant
kernel, from per-launch HIP event timing of the same workload), cpu_baseline
(the C oracle on this host, bounded sample) and per-stage kernel times.
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

# T, synthetic spec overrides
CONFIGS = {
    0: dict(T=1, name="moe_decode_b1", spec=dict(), layers=8),
    1: dict(T=8, name="moe_decode_b8", spec=dict(), layers=8),
}


def q4k_bytes(rows, cols):
    return rows * (cols // 256) * 144


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", type=int, default=0, choices=sorted(CONFIGS))
    ap.add_argument("--xbank", type=int, default=64)
    ap.add_argument("--graph-steps", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the MoE path is single-GPU; "
              "expert-parallel sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import orome_amd
    from orome_amd import _lib
    from orome_amd._lib import check, lib
    from orome_amd.moe import DeviceBuffer

    cf = CONFIGS[args.config]
    T, L = cf["T"], cf["layers"]
    H, E, K, M, S = 2048, 256, 8, 512, 512
    spec = orome_amd.make_spec(layers=L, H=H, E=E, K=K, M=M, S=S, seed=1234, **cf["spec"])
    print("[bench] config %d (%s): building %d synthetic layers" % (args.config, cf["name"], L),
          file=sys.stderr, flush=True)
    img = orome_amd.synth_gguf(spec)
    gm = orome_amd.MoEModel(image=img, max_tokens=max(T, 16))
    ctx = gm.ctx
    NX = args.xbank
    xs = [DeviceBuffer.from_array(ctx, orome_amd.synth_normal(77, i, T * H).reshape(T, H)) for i in range(NX)]
    hs = [DeviceBuffer.from_array(ctx, orome_amd.synth_normal(78, i, T * H).reshape(T, H)) for i in range(NX)]
    outs = [DeviceBuffer(ctx, T * H * 4) for _ in range(2)]

    def step(i):
        gm.forward(i % L, xs[i % NX], hs[i % NX], outs[i % 2], T)

    # unique experts per (layer, input) combination, for the algorithmic bytes
    combos = sorted({(i % L, i % NX) for i in range(args.graph_steps)})
    uniq = {}
    for (l, xi) in combos:
        gm.forward(l, xs[xi], hs[xi], outs[0], T)
        off = gm.debug_outputs(T)["offsets"]
        uniq[(l, xi)] = int(np.count_nonzero(np.diff(off.astype(np.int64))))
    u_mean = float(np.mean([uniq[(i % L, i % NX)] for i in range(args.graph_steps)]))

    # graphs: G steps per replay, plus a remainder graph so exactly K steps are timed
    G = min(args.graph_steps, args.steps)

    def capture(n, start=0):
        check(lib.orome_hip_capture_begin(ctx.handle), "capture")
        for i in range(n):
            step(start + i)
        ex = C.c_void_p()
        check(lib.orome_hip_capture_end(ctx.handle, C.byref(ex)), "capture_end")
        return ex

    g_main = capture(G)
    rem = args.steps % G
    g_rem = capture(rem) if rem else None
    reps = args.steps // G
    for _ in range(max(1, math.ceil(args.warmup / G))):
        check(lib.orome_hip_graph_launch(ctx.handle, g_main))
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        check(lib.orome_hip_graph_launch(ctx.handle, g_main))
    if g_rem:
        check(lib.orome_hip_graph_launch(ctx.handle, g_rem))
    ctx.sync()
    t1 = time.perf_counter()
    elapsed = t1 - t0
    K_steps = args.steps

    # per-kernel durations: the same steps, eager, with HIP events around each
    # launch on the context stream
    n_prof = min(args.steps, 1000)
    check(lib.orome_hip_stage_timing(ctx.handle, n_prof))
    for i in range(n_prof):
        step(i)
    tot = (C.c_float * 8)()
    cnt = (C.c_int * 8)()
    check(lib.orome_hip_stage_times(ctx.handle, tot, cnt, 8))
    check(lib.orome_hip_stage_timing(ctx.handle, 0))
    stage_us = {_lib.STAGES[i]: (tot[i] / cnt[i] * 1000.0 if cnt[i] else None) for i in range(8)}

    # algorithmic bytes (weights counted once per unique expert, activations once)
    w_exp = 3 * q4k_bytes(M, H)          # gate + up + down of one expert (Q4_K)
    w_sh = 3 * q4k_bytes(S, H)
    gu_bytes = (u_mean + 1) * 2 * q4k_bytes(M, H) + T * H * 4 + (T * K + T) * M * 2
    layer_bytes = (u_mean * w_exp + w_sh + E * H * 4 + H * 4 + T * H * 4 + 2 * T * H * 4)
    gu_us = stage_us["gate_up"]
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic_%s.json" % cf["name"])
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get("gate_up_hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        om = O.OracleModel(img)
        xh = [orome_amd.synth_normal(77, i, T * H).reshape(T, H) for i in range(NX)]
        hh = [orome_amd.synth_normal(78, i, T * H).reshape(T, H) for i in range(NX)]
        n = 0
        c0 = time.perf_counter()
        while time.perf_counter() - c0 < args.cpu_seconds:
            om.forward(n % L, xh[n % NX], hh[n % NX], omp=False)
            n += 1
        ct = time.perf_counter() - c0
        cpu = {"value": round(n * T / ct, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": "%d steps (%d tokens) of the same workload, scalar C oracle, 1 thread, "
                         "%.1f s" % (n, n * T, ct)}

    value = T * K_steps / elapsed
    out = {
        "metric": "MoE-layer tokens/s (B=%d decode, one MoE FFN block per step)" % T,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / K_steps * 1000, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded GGUF Q4_K per BASELINE config %d, %d rotating layers, %d inputs)"
                % (args.config, L, NX),
        "config": {"workload": cf["name"], "baseline_config": args.config, "tokens_per_step": T,
                   "hidden": H, "experts": E, "top_k": K, "expert_intermediate": M,
                   "shared_intermediate": S, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "gemv_gate_up", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes_per_launch": int(gu_bytes),
                     "avg_launch_us": round(gu_us, 3)},
        "layer": {"algorithmic_bytes_per_step": int(layer_bytes), "unique_experts_per_step": u_mean,
                  "gbs": round(layer_bytes * K_steps / elapsed / 1e9, 1),
                  "frac_of_hbm_peak": round(layer_bytes * K_steps / elapsed / 1e9 / HBM_PEAK_GBS, 4)},
        "stage_us": {k: (round(v, 3) if v is not None else None) for k, v in stage_us.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    lib.orome_hip_graph_destroy(g_main)
    if g_rem:
        lib.orome_hip_graph_destroy(g_rem)


if __name__ == "__main__":
    main()
