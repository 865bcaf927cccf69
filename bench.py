"""Benchmark of the INT4-G128-SYM projection path on one MI355X.

Headline (one JSON line on stdout): BASELINE config 1 -- the decode MLP
gate/up projection with the SiLU epilogue, M=1, K=5120, 2 x 17408 rows in
one interleaved packed-INT4 matrix (W_up = W_gate + 17408*2560 bytes),
17408 fp16 outputs.  One "step" = one launch over one batch.  `value` is
HBM GB/s of algorithmic bytes N*K/2 + N*(K/128)*2 + M*K*2 + M*N_out*2 per
step divided by the wall time per step, all inputs resident in HBM and the
weights rotated over enough copies (> 600 MB) that the 256 MB Infinity
Cache cannot hold them.  Launches are replayed from a HIP graph (how a
decode step is issued; the reference does the same with a SYCL graph,
src/targets/qwen3_8/decode_graph.cpp), so host launch cost is not timed.
Every timing first runs the GPU into its steady state: the requested warmup
launches, and at least 0.1 s of back-to-back launches (the first ~0.1 s of
work after an idle period measured up to 8 % slower per launch).

The other BASELINE configs are measured the same way under "suite"
(--quick skips them).  The CPU baseline is the oracle restatement of the
reference CPU loop, timed on this host's cores.

    python bench.py                       # default: N=1, all configs
    python bench.py --only cfg1 --no-cpu  # one config (profiling runs)
    python bench.py --calib-copy          # plain copy of known size (PMC scale)
    python bench.py --calib-dense-gemm    # hipBLASLt fp16 GEMM at the config 4 shape and two others
    python bench.py --calib-floor         # launch floor and vendor reads at the suite's byte counts
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0          # MI355X published HBM3E bandwidth
FP16_PEAK_TFLOPS = 2500.0       # MI355X published dense FP16 MFMA
MALL_BYTES = 256 << 20
ROTATE_MIN_BYTES = 600 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_config1_gate_up_m1.json")


def gemv_bytes(M, Nrows, K, Nout, out_bytes):
    """Algorithmic bytes of one INT4-G128 projection launch."""
    return Nrows * K // 2 + Nrows * (K // 128) * 2 + M * K * 2 + M * Nout * out_bytes


def cpu_count():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


class Rig:
    """Device buffers for one config: weight copies rotated per launch."""

    def __init__(self, torch, dev, Nrows, K, sigma, seed=0, copies=None):
        from xinfer_amd import synth
        W = synth.packed_weights(seed, Nrows, K)
        S = synth.scales(seed, Nrows, K, sigma)
        one = Nrows * K // 2 + Nrows * (K // 128) * 2
        self.copies = max(2, -(-ROTATE_MIN_BYTES // one)) if one < 4 * MALL_BYTES else 2
        if copies is not None:
            self.copies = copies
        w0 = torch.from_numpy(W).to(dev)
        s0 = torch.from_numpy(S).view(torch.float16).to(dev)
        self.W = [w0] + [w0.clone() for _ in range(self.copies - 1)]
        self.S = [s0] + [s0.clone() for _ in range(self.copies - 1)]


MIN_WARM_S = 0.1  # the GPU reaches its steady clock after ~0.1 s of back-to-back work


def _time_eager(torch, launch, steps, warmup, copies):
    t0 = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t0 < MIN_WARM_S:
        launch(i % copies)
        i += 1
        if i % 64 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(st)
    for i in range(steps):
        launch(i % copies)
    e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall / steps, e0.elapsed_time(e1) * 1e-3 / steps


def _time_graph(torch, launch, steps, warmup, copies):
    per = copies * max(1, 32 // copies)          # launches per graph
    for i in range(per):
        launch(i % copies)                          # warm up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(per):
                launch(i % copies)
    reps = max(1, steps // per)
    t0 = time.perf_counter()
    r = 0
    while r < max(1, warmup // per) or time.perf_counter() - t0 < MIN_WARM_S:
        g.replay()
        r += 1
        if r % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(reps):
        g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    n = reps * per
    return wall / n, e0.elapsed_time(e1) * 1e-3 / n, n


def time_exact(torch, launch, steps, warmup, copies):
    """The headline timing: exactly `steps` launches (rotating the weight
    copies) captured in one HIP graph.  Untimed: `warmup` launches' worth of
    replays (and at least MIN_WARM_S of work).  Timed: one replay of the
    `steps` launches, synchronized on both sides, by the host clock and by
    events on the replay stream.  Then 9 more replays, each timed by events:
    their median per launch is reported beside the mean of the timed one.
    Also returns the event time of one launch from cold: code loaded, the
    Infinity Cache flushed by a 512 MiB fill, the GPU idle for 50 ms."""
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    launch(1 % copies)  # loads the code object
    flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    flush.fill_(1)
    torch.cuda.synchronize()
    del flush
    time.sleep(0.05)
    e0.record(st)
    launch(0)
    e1.record(st)
    torch.cuda.synchronize()
    cold = e0.elapsed_time(e1) * 1e-3
    for i in range(copies):
        launch(i % copies)                          # warm up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                launch(i % copies)
    t0 = time.perf_counter()
    done = 0
    while done < warmup or time.perf_counter() - t0 < MIN_WARM_S:
        g.replay()
        done += steps
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(st)
    g.replay()
    e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev = e0.elapsed_time(e1) * 1e-3
    per = []
    for _ in range(9):
        e0.record(st)
        g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) * 1e-3 / steps)
    per.sort()
    return wall / steps, ev / steps, per[len(per) // 2], cold


def time_launches(torch, launch, steps, warmup, copies, graph=False):
    """(wall s/step, event s/step) for `steps` launches rotating weight copies.
    graph=True captures one rotation into a HIP graph and times replays.
    The events are recorded on the stream the kernels run on."""
    if graph:
        w, e, _ = _time_graph(torch, launch, steps, warmup, copies)
        return w, e
    return _time_eager(torch, launch, steps, warmup, copies)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    # ~0.15 s of untimed launches: the first ~0.1 s of back-to-back work on
    # the box ran up to 8 % slower per launch (clock ramp), measured
    ap.add_argument("--warmup", type=int, default=8000)
    ap.add_argument("--quick", action="store_true", help="headline config only")
    ap.add_argument("--only", default="", help="comma list: cfg1,ns,cfg0,cfg2,fused,norm,layer,crc,cfg3,cfg4")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-exact", action="store_true",
                    help="skip config 4 on the exact-dequant route (a child process)")
    ap.add_argument("--eager", action="store_true", help="time eager launches, not graph replay")
    ap.add_argument("--calib-copy", action="store_true",
                    help="run a plain 256 MiB device copy 20x (PMC calibration) and exit")
    ap.add_argument("--calib-floor", action="store_true",
                    help="graph-replayed launch floor and torch reductions over the suite's byte counts")
    ap.add_argument("--calib-dense-gemm", action="store_true",
                    help="time torch.matmul (hipBLASLt) fp16 X @ W^T at the config 4 shape and exit")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build's INT4 projection path is a "
              "single-GPU kernel (multi-GPU sharding is design-only); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from xinfer_amd import ops, synth
    from xinfer_amd._lib import load_library
    load_library()
    dev = torch.device("cuda:0")
    log = lambda *a: print(*a, file=sys.stderr, flush=True)  # noqa: E731

    if args.calib_copy:
        n = 256 << 20
        a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(20):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copied {n} bytes x 20")
        return

    if args.calib_floor:
        # The fixed cost of a graph-replayed launch (an empty kernel) and the
        # time of a kernel that only reads B bytes (grid-stride 16-byte loads,
        # libxinfer_calib.so) at the byte counts of the suite's shapes,
        # buffers rotated past the Infinity Cache like the projections: what
        # a projection of the same bytes can reach on this GPU.
        import ctypes
        cal = ctypes.CDLL(os.path.join(ROOT, "xinfer_amd", "lib", "libxinfer_calib.so"))
        cal.xinfer_calib_empty.argtypes = [ctypes.c_void_p]
        cal.xinfer_calib_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                          ctypes.c_int]
        sink = torch.zeros(4, dtype=torch.int32, device=dev)

        def empty(i):
            assert cal.xinfer_calib_empty(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
        w, e = time_launches(torch, empty, 4000, 4000, 1, graph=True)
        print(json.dumps({"calib": "launch_floor_empty_kernel", "us": round(e * 1e6, 3)}), flush=True)
        for name, nbytes in (("cfg0_qproj_m1", 6144 * 5120 // 2), ("cfg2_down_m1", 5120 * 17408 // 2),
                             ("cfg1_gate_up_m1", 2 * 17408 * 5120 // 2),
                             ("cfg3_lm_head_m1", 151936 * 5120 // 2)):
            copies = max(1, -(-ROTATE_MIN_BYTES // nbytes))
            bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(copies)]
            for blocks in (0, 1024):
                def rd(i, bufs=bufs, nbytes=nbytes, blocks=blocks):
                    assert cal.xinfer_calib_read(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                                 ctypes.c_void_p(bufs[i].data_ptr()), nbytes,
                                                 ctypes.c_void_p(sink.data_ptr()), blocks) == 0
                w, e = time_launches(torch, rd, max(copies, 400), max(copies, 400), copies, graph=True)
                print(json.dumps({"calib": "read_only_kernel", "shape": name, "bytes": nbytes,
                                  "blocks": blocks or "8 per CU", "us": round(e * 1e6, 3),
                                  "GBps": round(nbytes / e / 1e9, 1), "frac_hbm": round(nbytes / e / 1e9 / HBM_PEAK_GBPS, 4),
                                  "copies": copies}), flush=True)
            del bufs
        return

    if args.calib_dense_gemm:
        # Reference points for the prefill GEMM: the vendor library's dense
        # fp16 GEMM (no dequantisation) in the same weight layout ([N][K],
        # row-major), weights rotated past the Infinity Cache: the config 4
        # shape, twice its M, and a large square GEMM.
        for M, N, K in ((512, 17408, 5120), (1024, 17408, 5120), (8192, 8192, 8192)):
            copies = max(1, -(-ROTATE_MIN_BYTES // (N * K * 2)))
            X = torch.randn(M, K, dtype=torch.float16, device=dev)
            Ws = [torch.randn(N, K, dtype=torch.float16, device=dev) for _ in range(copies)]
            Y = torch.empty(M, N, dtype=torch.float16, device=dev)
            fn = lambda i, X=X, Ws=Ws, Y=Y: torch.matmul(X, Ws[i].t(), out=Y)  # noqa: E731
            steps = max(copies, min(args.steps, int(2e13 // (2 * M * N * K))))
            w, e = time_launches(torch, fn, steps, max(copies, args.warmup // 20), copies, graph=True)
            tf = 2.0 * M * N * K / e / 1e12
            print(json.dumps({"calib": "dense_fp16_gemm_hipblaslt", "M": M, "N": N, "K": K,
                              "us": round(e * 1e6, 2), "TFLOPs": round(tf, 1),
                              "frac_fp16_mfma": round(tf / FP16_PEAK_TFLOPS, 4),
                              "weight_copies": copies}), flush=True)
            del X, Ws, Y
        return

    only = set(x for x in args.only.split(",") if x)
    want = lambda k: (not only) or (k in only)  # noqa: E731
    graph = not args.eager

    # ---------------- headline: config 1, fused gate/up + SiLU, M=1 ----------------
    M, N, K = 1, 17408, 5120
    nbytes = gemv_bytes(M, 2 * N, K, N, 2)
    head = None
    if want("cfg1"):
        rig = Rig(torch, dev, 2 * N, K, 0.02)
        X = torch.from_numpy(synth.activations(0, M, K)).view(torch.float16).to(dev)
        Y = torch.empty((M, N), dtype=torch.float16, device=dev)

        def launch_cfg1(i):
            W, S = rig.W[i], rig.S[i]
            ops.mlp_gate_up_swiglu_int4(Y, X, W[:N], S[:N], W[N:], S[N:], M, N, K)

        if graph:
            wall_step, ev_step, ev_med, cold = time_exact(torch, launch_cfg1, args.steps, args.warmup,
                                                          rig.copies)
        else:
            wall_step, ev_step = time_launches(torch, launch_cfg1, args.steps, args.warmup,
                                               rig.copies, graph=False)
            ev_med, cold = ev_step, None
        head = (wall_step, ev_step, rig.copies, ev_med, cold)
        log(f"config 1: M={M} K={K} N=2x{N}, {rig.copies} weight copies, {args.steps} launches timed, "
            f"wall {wall_step*1e6:.2f} us/step, events {ev_step*1e6:.2f} us/launch "
            f"(median of 9 more replays {ev_med*1e6:.2f}), {nbytes/ev_step/1e9:.0f} GB/s; "
            f"first launch (cold) {cold*1e6 if cold else float('nan'):.1f} us")
        del rig

    suite = {} if args.quick else run_suite(torch, dev, ops, synth, args, log, want, graph)

    cpu = None
    if not args.no_cpu and head is not None:
        cpu = cpu_baseline(nbytes, log)

    if head is None:
        print(json.dumps({"suite": suite}), flush=True)
        return
    wall_step, ev_step, copies, ev_med, cold = head
    value = nbytes / wall_step / 1e9
    achieved = nbytes / ev_step / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        traffic = t.get("hbm_bytes_per_launch")
    line = {
        "metric": "INT4 GEMV HBM GB/s (% of MI355X peak) at M=1; prefill GEMM TFLOP/s at M=512",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_step * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 x f16 -> f32 accumulate",
        "data": "synthetic (SplitMix64 seed 0: uniform int4, |N(0,0.02)|/7 fp16 scales, N(0,1) fp16 x)",
        "config": {"workload": "BASELINE config 1: fused gate/up SiLU decode GEMV",
                   "M": M, "K": K, "N": f"2x{N}", "group_size": 128,
                   "weight_copies_rotated": copies,
                   "launch": "hip graph replay" if graph else "eager"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic,
                     "traffic_source": "profiles/traffic_config1_gate_up_m1.json: committed rocprofv3 --pmc "
                                       "FETCH_SIZE + WRITE_SIZE of this kernel, scaled by a plain copy "
                                       "of known size (not measured in this run)",
                     "kernel": "xhip::gemv_pair_int4_kernel<P=5,f16,SWIGLU> (row pairs; each wave streams its gate pairs, then the same up pairs)",
                     "algorithmic_bytes_per_launch": nbytes,
                     "avg_launch_us": round(ev_step * 1e6, 3),
                     "median_launch_us_9_replays": round(ev_med * 1e6, 3),
                     "cold_first_launch_us": round(cold * 1e6, 2) if cold else None},
        "cpu_baseline": cpu,
        "suite": suite,
    }
    print(json.dumps(line), flush=True)


def run_suite(torch, dev, ops, synth, args, log, want, graph):
    out = {}
    steps = max(64, min(args.steps, 512))
    warm = min(args.warmup, 32)

    def record(name, d):
        out[name] = d
        log(f"  {name}: {d}")

    def gemv_cfg(name, M, N, K, sigma=0.02):
        rig = Rig(torch, dev, N, K, sigma)
        X = torch.from_numpy(synth.activations(0, M, K)).view(torch.float16).to(dev)
        Y = torch.empty((M, N), dtype=torch.float16, device=dev)
        fn = lambda i: ops.linear_int4(Y, X, rig.W[i], rig.S[i], None, M, N, K)  # noqa: E731
        w, e = time_launches(torch, fn, steps, warm, rig.copies, graph=graph)
        b = gemv_bytes(M, N, K, N, 2)
        record(name, {"M": M, "N": N, "K": K, "us": round(e * 1e6, 3),
                      "GBps": round(b / e / 1e9, 1), "frac_hbm": round(b / e / 1e9 / HBM_PEAK_GBPS, 4)})

    if want("ns"):
        gemv_cfg("northstar_gemv_m1_n34816_k5120", 1, 34816, 5120)
    if want("cfg0"):
        gemv_cfg("cfg0_qproj_m1_n6144_k5120", 1, 6144, 5120)
    if want("cfg2"):
        for m in (1, 2, 4, 8):
            gemv_cfg(f"cfg2_down_m{m}_n5120_k17408", m, 5120, 17408)

    if want("fused"):  # decode projections of forward_layer (forward.cpp:117-125, 237-247)
        K = 5120
        for name, Ns in (("qkv", (12288, 1024, 1024)), ("la_in_proj", (10240, 6144, 48, 48))):
            rigs = [Rig(torch, dev, N, K, 0.02, seed=i) for i, N in enumerate(Ns)]
            copies = min(r.copies for r in rigs)
            X = torch.from_numpy(synth.activations(0, 1, K)).view(torch.float16).to(dev)
            Ys = [torch.empty((1, N), dtype=torch.float16, device=dev) for N in Ns]
            def fn(i, rigs=rigs, Ys=Ys, Ns=Ns, X=X):
                ds = [ops.FusedProjectionDesc(Y, r.W[i], r.S[i], None, N) for Y, r, N in zip(Ys, rigs, Ns)]
                ops.linear_int4_fused(X, ds, len(ds), 1, K)
            w, e = time_launches(torch, fn, steps, warm, copies, graph=graph)
            b = sum(gemv_bytes(1, N, K, N, 2) for N in Ns) - (len(Ns) - 1) * K * 2
            record(f"fused_{name}_m1_k5120", {"M": 1, "N": list(Ns), "K": K, "us": round(e * 1e6, 3),
                                             "GBps": round(b / e / 1e9, 1),
                                             "frac_hbm": round(b / e / 1e9 / HBM_PEAK_GBPS, 4)})
            del rigs
        gemv_cfg("splitk_small_n48_m1_k5120", 1, 48, 5120)

    if want("norm"):   # RMSNorm prologue / residual epilogue, fused vs separate launches
        K, Ns = 5120, (12288, 1024, 1024)
        rigs = [Rig(torch, dev, N, K, 0.02, seed=i) for i, N in enumerate(Ns)]
        copies = min(r.copies for r in rigs)
        nw = torch.linspace(0.5, 1.5, K, dtype=torch.float32, device=dev)
        for M in (1, 2, 3, 4, 6, 8):
            X = torch.from_numpy(synth.activations(0, M, K)).view(torch.float16).to(dev)
            Xn = torch.empty_like(X)
            ws = torch.empty(max(1, M * K * 2), dtype=torch.uint8, device=dev)
            Ys = [torch.empty((M, N), dtype=torch.float16, device=dev) for N in Ns]

            def fused(i, rigs=rigs, Ys=Ys, X=X, M=M, ws=ws):
                ds = [ops.FusedProjectionDesc(Y, r.W[i], r.S[i], None, N) for Y, r, N in zip(Ys, rigs, Ns)]
                ops.rmsnorm_linear_int4_fused(X, nw, 1e-6, ds, 3, M, K, workspace=ws)

            def separate(i, rigs=rigs, Ys=Ys, X=X, Xn=Xn, M=M):
                ops.rmsnorm(Xn, X, nw, M, K, 1e-6)
                ds = [ops.FusedProjectionDesc(Y, r.W[i], r.S[i], None, N) for Y, r, N in zip(Ys, rigs, Ns)]
                ops.linear_int4_fused(Xn, ds, 3, M, K)
            _, ef = time_launches(torch, fused, steps, warm, copies, graph=graph)
            _, es = time_launches(torch, separate, steps, warm, copies, graph=graph)
            record(f"rmsnorm_qkv_m{M}_k5120", {"M": M, "N": list(Ns), "K": K, "us_fused": round(ef * 1e6, 3),
                                               "us_separate": round(es * 1e6, 3)})
        del rigs
        N, K = 17408, 5120                     # gate/up SwiGLU with the input norm
        rig = Rig(torch, dev, 2 * N, K, 0.02)
        for M in (2, 4, 8):
            X = torch.from_numpy(synth.activations(0, M, K)).view(torch.float16).to(dev)
            Xn = torch.empty_like(X)
            ws = torch.empty(M * K * 2, dtype=torch.uint8, device=dev)
            Y = torch.empty((M, N), dtype=torch.float16, device=dev)

            def fused_g(i, X=X, Y=Y, M=M, ws=ws):
                W, S = rig.W[i], rig.S[i]
                ops.rmsnorm_mlp_gate_up_swiglu_int4(Y, X, nw, 1e-6, W[:N], S[:N], W[N:], S[N:], M, N, K,
                                                    workspace=ws)

            def separate_g(i, X=X, Xn=Xn, Y=Y, M=M):
                ops.rmsnorm(Xn, X, nw, M, K, 1e-6)
                W, S = rig.W[i], rig.S[i]
                ops.mlp_gate_up_swiglu_int4(Y, Xn, W[:N], S[:N], W[N:], S[N:], M, N, K)
            _, ef = time_launches(torch, fused_g, steps, warm, rig.copies, graph=graph)
            _, es = time_launches(torch, separate_g, steps, warm, rig.copies, graph=graph)
            record(f"rmsnorm_gate_up_m{M}_n17408_k5120", {"M": M, "N": N, "K": K, "us_fused": round(ef * 1e6, 3),
                                                         "us_separate": round(es * 1e6, 3)})
        del rig
        N, K = 5120, 6144                      # o_proj of a full-attention layer
        rig = Rig(torch, dev, N, K, 0.02)
        for M in (1, 4):
            X = torch.from_numpy(synth.activations(0, M, K)).view(torch.float16).to(dev)
            R = torch.zeros((M, N), dtype=torch.float16, device=dev)
            Y = torch.empty((M, N), dtype=torch.float16, device=dev)

            def fused_r(i, X=X, R=R, M=M):
                ops.linear_int4_residual(R, X, rig.W[i], rig.S[i], None, M, N, K)

            def separate_r(i, X=X, R=R, Y=Y, M=M):
                ops.linear_int4(Y, X, rig.W[i], rig.S[i], None, M, N, K)
                ops.add_inplace(R, Y, M * N)
            _, ef = time_launches(torch, fused_r, steps, warm, rig.copies, graph=graph)
            _, es = time_launches(torch, separate_r, steps, warm, rig.copies, graph=graph)
            record(f"residual_oproj_m{M}_n5120_k6144", {"M": M, "N": N, "K": K, "us_fused": round(ef * 1e6, 3),
                                                         "us_separate": round(es * 1e6, 3)})
        del rig

    if want("layer"):  # one decode layer's projection sequence (forward.cpp:112-125, 229, 273-290)
        H, Q, KV, AO, I = 5120, 12288, 1024, 6144, 17408
        layers = []
        for c in range(2):  # two copies (372 MB > the 256 MB Infinity Cache), alternated
            mk = lambda i, n, k, c=c: Rig(torch, dev, n, k, 0.02, seed=10 * c + i, copies=1)  # noqa: E731
            layers.append(dict(q=mk(0, Q, H), k=mk(1, KV, H), v=mk(2, KV, H), o=mk(3, H, AO),
                               g=mk(4, I, H), u=mk(5, I, H), d=mk(6, H, I)))
        lnw = [torch.linspace(0.5, 1.5, H, dtype=torch.float32, device=dev) for _ in range(2)]
        nbytes = sum(gemv_bytes(1, r.W[0].shape[0], r.W[0].shape[1] * 2, 0, 0)
                     for r in layers[0].values())
        for M in (1, 4, 8):  # decode, and the speculative verify rows (forward.cpp:729-732)
            f16 = dict(dtype=torch.float16, device=dev)
            resid = torch.from_numpy(synth.activations(0, M, H)).view(torch.float16).to(dev)
            bq, bk, bv = (torch.empty((M, n), **f16) for n in (Q, KV, KV))
            attn = torch.from_numpy(synth.activations(1, M, AO)).view(torch.float16).to(dev)
            act = torch.empty((M, I), **f16)
            ws = torch.empty(M * H * 2, dtype=torch.uint8, device=dev)  # normalised rows (M >= 2)

            def layer_step(i, M=M, resid=resid, bq=bq, bk=bk, bv=bv, attn=attn, act=act, ws=ws):
                Lr = layers[i % 2]
                ds = [ops.FusedProjectionDesc(Y, Lr[n].W[0], Lr[n].S[0], None, N)
                      for Y, n, N in ((bq, "q", Q), (bk, "k", KV), (bv, "v", KV))]
                ops.rmsnorm_linear_int4_fused(resid, lnw[0], 1e-6, ds, 3, M, H, workspace=ws)
                ops.linear_int4_residual(resid, attn, Lr["o"].W[0], Lr["o"].S[0], None, M, H, AO)
                ops.rmsnorm_mlp_gate_up_swiglu_int4(act, resid, lnw[1], 1e-6, Lr["g"].W[0], Lr["g"].S[0],
                                                    Lr["u"].W[0], Lr["u"].S[0], M, I, H, workspace=ws)
                ops.linear_int4_residual(resid, act, Lr["d"].W[0], Lr["d"].S[0], None, M, H, I)
            _, eg = time_launches(torch, layer_step, 256, warm, 2, graph=True)
            _, ee = time_launches(torch, layer_step, 256, warm, 2, graph=False)
            record(f"decode_layer_projections_m{M}", {
                "M": M, "launches_per_step": 4, "weight_bytes": nbytes,
                "us_graph": round(eg * 1e6, 2), "us_eager": round(ee * 1e6, 2),
                "GBps_graph": round(nbytes / eg / 1e9, 1),
                "frac_hbm_graph": round(nbytes / eg / 1e9 / HBM_PEAK_GBPS, 4)})
        del layers

    if want("crc"):    # .xinfer section verification on the device (GPU CRC-64)
        import ctypes
        from xinfer_amd import _lib
        L = _lib.load_library()
        n = 256 << 20
        bufs = [torch.randint(0, 256, (n,), dtype=torch.uint8, device=dev) for _ in range(3)]
        crc_out = torch.zeros(1, dtype=torch.int64, device=dev)
        scratch = torch.empty(L.xinfer_crc64_device_scratch_bytes(n), dtype=torch.uint8, device=dev)

        def crc(i):
            st = torch.cuda.current_stream().cuda_stream
            _lib.check("xinfer_crc64_device", L.xinfer_crc64_device(
                ctypes.c_void_p(st), ctypes.c_void_p(bufs[i].data_ptr()), n, ctypes.c_void_p(crc_out.data_ptr()),
                ctypes.c_void_p(scratch.data_ptr()), scratch.numel()))
        w, e = time_launches(torch, crc, 48, 6, len(bufs), graph=graph)
        record("artifact_crc64_device_256MiB", {"bytes": n, "us": round(e * 1e6, 2),
                                                "GBps": round(n / e / 1e9, 1),
                                                "frac_hbm": round(n / e / 1e9 / HBM_PEAK_GBPS, 4)})
        del bufs

    if want("cfg3"):   # LM head + argmax (ids only, logits not stored)
        N, K = 151936, 5120
        rig = Rig(torch, dev, N, K, 0.01)
        for M in (1, 8):
            X = torch.from_numpy(synth.activations(0, M, K)).view(torch.float16).to(dev)
            ids = torch.empty(M, dtype=torch.int32, device=dev)
            scr = torch.empty(ops.lm_head_argmax_scratch_size(M, N, K), dtype=torch.uint8, device=dev)
            fn = lambda i: ops.lm_head_argmax_int4(ids, None, X, rig.W[i], rig.S[i], M, N, K,  # noqa
                                                    scratch=scr)
            w, e = time_launches(torch, fn, steps, warm, rig.copies, graph=graph)
            b = gemv_bytes(M, N, K, 0, 0) + M * 4
            record(f"cfg3_lmhead_argmax_m{M}", {"M": M, "N": N, "K": K, "us": round(e * 1e6, 3),
                                                "GBps": round(b / e / 1e9, 1),
                                                "frac_hbm": round(b / e / 1e9 / HBM_PEAK_GBPS, 4)})
        del rig

    if want("cfg4"):   # chunked-prefill GEMM M=512
        M, N, K = 512, 17408, 5120
        rig = Rig(torch, dev, N, K, 0.02)
        X = torch.from_numpy(synth.activations(0, M, K)).view(torch.float16).to(dev)
        Y = torch.empty((M, N), dtype=torch.float16, device=dev)
        fn = lambda i: ops.linear_int4(Y, X, rig.W[i], rig.S[i], None, M, N, K)  # noqa: E731
        w, e = time_launches(torch, fn, max(32, steps // 4), 8, rig.copies, graph=graph)
        fl = 2 * M * N * K
        exact_route = os.environ.get("XINFER_GEMM_EXACT") == "1"
        record("cfg4_prefill_exact_dequant_m512_n17408_k5120" if exact_route else "cfg4_prefill_m512_n17408_k5120",
               {"M": M, "N": N, "K": K, "us": round(e * 1e6, 2), "TFLOPs": round(fl / e / 1e12, 1),
                "frac_fp16_mfma": round(fl / e / 1e12 / FP16_PEAK_TFLOPS, 4),
                "kernel": ("xhip::gemm_int4_mfma_kernel<EXACT> (exact q, FP32 group scale; 128-row blocks)"
                           if exact_route else
                           "xhip::gemm_ws_int4_kernel (256x136 blocks; 4 MFMA waves copying their own X "
                           "rows, 4 weight-decode waves; B = fp16(q*s))")})
        if not exact_route and not args.no_exact:
            # the same projection with the reference's dequantisation (exact
            # integer q, FP32 group scale) on the other GEMM kernel, in a
            # child process (the route is chosen from the environment once)
            env = dict(os.environ, XINFER_GEMM_WS="0", XINFER_GEMM_EXACT="1")
            r = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "cfg4", "--no-cpu",
                                "--steps", str(args.steps), "--warmup", str(args.warmup)]
                               + (["--eager"] if args.eager else []),
                               capture_output=True, text=True, env=env, timeout=300)
            try:
                sub = json.loads(r.stdout.strip().splitlines()[-1])["suite"]
                for k, v in sub.items():
                    record(k, v)
            except Exception as ex:  # noqa: BLE001 (reported, not fatal to the headline)
                log(f"  exact-dequant child failed: {ex}: {r.stderr[-500:]}")
    return out


def cpu_baseline(nbytes, log):
    """Oracle restatement of the reference CPU loop (double accumulate) on
    the full config-1 step, repeated for >= ~10 s per thread setting."""
    try:
        import oracle
        oracle.lib()
    except Exception as e:  # the oracle library travels prebuilt; report if absent
        log(f"cpu baseline unavailable: {e}")
        return None
    from xinfer_amd import synth
    M, N, K = 1, 17408, 5120
    W = synth.packed_weights(0, 2 * N, K)
    S = synth.scales(0, 2 * N, K)
    X = oracle.f16_to_f32(synth.activations(0, M, K))
    res = {}
    for threads in (cpu_count(), 1):
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle.swiglu_int4(X, W[:N], S[:N], W[N:], S[N:], M, N, K, nthreads=threads)
            reps += 1
            if time.perf_counter() - t0 >= 10.0:
                break
        dt = (time.perf_counter() - t0) / reps
        res[threads] = (nbytes / dt / 1e9, dt, reps)
        log(f"  cpu oracle {threads} thread(s): {dt*1e3:.1f} ms/step, {reps} reps")
    cores = cpu_count()
    v, dt, reps = res[cores]
    model = ""
    try:
        info = {}
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ":" in ln:
                    k_, v_ = ln.split(":", 1)
                    info.setdefault(k_.strip(), v_.strip())
                if not ln.strip() and info:
                    break
        model = info.get("model name", "")
        # family / model / stepping identify the part when the name is generic
        model += " (family %s, model %s, stepping %s)" % (info.get("cpu family", "?"), info.get("model", "?"),
                                                         info.get("stepping", "?"))
    except OSError:
        pass
    log(f"  cpu: {model} ({os.cpu_count()} logical cpus on the host, {cores} used)")
    return {"value": round(v, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu_model": model, "host_nproc": os.cpu_count(),
            "sample": f"full config-1 step (M=1, K=5120, 2x17408 rows) x {reps} reps, "
                      f"OpenMP over {cores} threads; single-thread: "
                      f"{res[1][0]:.3f} GB/s ({res[1][1]*1e3:.0f} ms/step)",
            "ms_per_step": round(dt * 1e3, 2)}


if __name__ == "__main__":
    main()
