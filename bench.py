"""Benchmark of the MI355X quantized decode path (BASELINE.json metric:
"MoE decode FFN: effective HBM GB/s (% of peak) + us/layer at M=1 and M=8").

Workload (value): BASELINE config 3 -- one Qwen3.5-35B-A3B-shaped MoE decode
FFN layer at M=1: hidden 2048, 256 experts (gate/up 512x2048, down 2048x512,
Q4_0), top-8 + one Q4_0 shared expert, f32 router 256x2048.  A step is one
layer call (router -> top-k -> gate/up+SiLU -> down -> weighted sum + shared)
on one token.  value = selected-expert bytes per step (8 x 1,769,472 B) /
time per step.  Weights are synthetic N(0, 0.02), seeded, quantized on the
device; each step uses a different (layer copy, token) slot so that the bytes
come from HBM and not from the 256 MB Infinity Cache.  Timed as one HIP graph
of exactly K steps between events, after W warm-up steps.

Also reported (extra): M=8 IQ3_S layer (config 4, uniform and Zipf routing),
one token through the IQ3_S layers with a Q8_0 and with a Q5_K shared expert
(the reference model's types),
the 512-token Q4_0 prefill chunk (config 5, int8 MFMA), the Q4_0 151936x2048
head GEMV (config 2), the Q8_0 4096x2048 GEMV (config 1),
per-kernel times and the roofline of the dominant kernel, and the CPU
baseline (the C restatement in oracle/, timed on this host).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
Q4_0, Q8_0, IQ3_S = 2, 8, 21


def row_bytes(t, ncols):
    return {Q8_0: ncols // 32 * 34, Q4_0: ncols // 32 * 18, IQ3_S: ncols // 256 * 110}[t]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="only the headline workload")
    ap.add_argument("--no-ncmoe", action="store_true", help="skip the host expert path (ncmoe) figures")
    ap.add_argument("--cpu-seconds", type=float, default=6.0, help="CPU baseline budget (about a tenth per figure)")
    ap.add_argument("--pmc", action="store_true", help="light mode for rocprofv3 --pmc runs")
    ap.add_argument("--pmc-workload", choices=["m1", "m8", "prefill", "prefill_iq3s", "head", "q5k"], default="m1",
                    help="workload of the --pmc light mode")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="run one device copy of this many MiB at the end (calibrates PMC byte counters)")
    return ap.parse_args()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py: this build runs on one GPU; --gpus above 1 is not supported", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from chimere_amd import ggml_gpu as G
    from chimere_amd.moe import MoeLayer

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    H, F, E, K = 2048, 512, 256, 8

    def qmat(t, rows, cols, n, g):
        out = torch.empty(n, rows * row_bytes(t, cols), dtype=torch.uint8, device=dev)
        step = max(1, (1 << 28) // (rows * cols))   # experts per launch: 1 GiB of f32 staging at most
        for i in range(0, n, step):
            m = min(step, n - i)
            wf = torch.randn(m * rows, cols, generator=g, device=dev) * 0.02
            G.quantize_weights(t, wf, out[i:i + m])
            del wf
        return out

    def make_layer(seed, t, st, E=256, H=2048, F=512, K=8, bias=None):
        g = torch.Generator(device=dev).manual_seed(seed)
        router = torch.randn(E, H, generator=g, device=dev) * 0.02
        gate, up, down = qmat(t, F, H, E, g), qmat(t, F, H, E, g), qmat(t, H, F, E, g)
        sh = (qmat(st, F, H, 1, g)[0], qmat(st, F, H, 1, g)[0], qmat(st, H, F, 1, g)[0])
        return MoeLayer(router, gate, up, down, t, K, shared=sh, shared_type=st, logit_bias=bias)

    def step_layers(base, n, seed, st, shared=None, bias=None):
        """n layers, one per step: each with its own router and shared expert
        (so that no step finds them in the memory-side cache after an earlier
        step of the same replay), the routed experts of base[i % len(base)].
        shared(i, g) -> the step's shared-expert matrices (default: N(0, 0.02)
        quantized to st)."""
        out = []
        for i in range(n):
            L = base[i % len(base)]
            g = torch.Generator(device=dev).manual_seed(seed + i)
            router = torch.randn(E, H, generator=g, device=dev) * 0.02
            sh = shared(i, g) if shared else (qmat(st, F, H, 1, g)[0], qmat(st, F, H, 1, g)[0], qmat(st, H, F, 1, g)[0])
            out.append(MoeLayer(router, L.tensors[1], L.tensors[2], L.tensors[3], L.expert_type, K, shared=sh,
                                shared_type=st, logit_bias=bias))
        return out

    def graph_time(fn_list, reps=5, flush=None):
        """Capture fn_list (callables, each one step) in one HIP graph; return
        the median over `reps` timed replays of the seconds per replay.  With
        `flush`, it runs (untimed) before every timed replay, so that weights
        come from HBM and not from the 256 MB memory-side cache."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for f in fn_list[: min(4, len(fn_list))]:
                f()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for f in fn_list:
                f()
        gr.replay()                         # warm replay
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            if flush is not None:
                flush()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            gr.replay()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / 1e3)
        return float(np.median(times)), gr

    if args.pmc:
        # counter-collection mode (rocprofv3 --pmc serialises every dispatch):
        # one layer, a few eager layer calls, then the calibration copy
        wl = args.pmc_workload
        print(f"bench.py --pmc: building the {wl} workload", flush=True)
        if wl == "head":
            V = 151936
            g = torch.Generator(device=dev).manual_seed(2)
            head = qmat(Q4_0, V, H, 1, g)[0]
            xq = torch.empty(G.q8_1_row_bytes(H), dtype=torch.uint8, device=dev)
            G.ggml_gpu_quantize_q8_1(torch.randn(H, generator=g, device=dev), xq, H)
            y = torch.empty(V, device=dev)
            for i in range(args.steps):
                G.ggml_gpu_gemv_q4_0_q8(head, xq, y, V, H)
        elif wl == "q5k":
            # the Q5_K GEMV (the reference model's shared-expert type) at 16384 x 4096,
            # random valid blocks as in the timed leg
            Rk, Ck = 16384, 4096
            g = torch.Generator(device=dev).manual_seed(2)
            wk = torch.randint(0, 256, (Rk * (Ck // 256 * 176),), dtype=torch.uint8, device=dev, generator=g)
            xk = torch.empty(G.q8_1_row_bytes(Ck), dtype=torch.uint8, device=dev)
            G.ggml_gpu_quantize_q8_1(torch.randn(Ck, generator=g, device=dev), xk, Ck)
            yk = torch.empty(Rk, device=dev)
            for i in range(args.steps):
                G.ggml_gpu_gemv_q5k_q8(wk, xk, yk, Rk, Ck)
        else:
            L = make_layer(100, *((IQ3_S, Q8_0) if wl in ("m8", "prefill_iq3s") else (Q4_0, Q4_0)))
            M = {"m1": 1, "m8": 8, "prefill": 512, "prefill_iq3s": 512}[wl]
            xs = torch.randn(args.steps, M, H, device=dev)
            out = torch.empty(M, H, device=dev)
            for i in range(args.steps):
                if wl.startswith("prefill"):
                    L.prefill(xs[i], out=out)
                else:
                    L.forward(xs[i], out=out)
        torch.cuda.synchronize()
        print(f"bench.py --pmc: {args.steps} {wl} calls done", flush=True)
        if args.calib_copy_mb:
            src = torch.empty(args.calib_copy_mb << 18, dtype=torch.float32, device=dev).fill_(1.0)
            dst = torch.empty_like(src)
            torch.cuda.synchronize()
            dst.copy_(src)
            torch.cuda.synchronize()
        print(json.dumps({"pmc_mode": True, "steps": args.steps, "calib_copy_mib": args.calib_copy_mb}), flush=True)
        return
    sel_bytes = K * (2 * F * row_bytes(Q4_0, H) + H * row_bytes(Q4_0, F))       # 14,155,776
    expert_bytes = sel_bytes // K
    all_bytes = sel_bytes + expert_bytes + E * H * 4 + H * 4 * 2                  # + shared, router, x, out

    # ---------------- headline: config 3, M=1 Q4_0.  Every step of the timed
    # graph is its own layer: its own router, shared expert and token, the
    # routed experts from one of up to 8 copies of the 256-expert tensors
    # (453 MB each), so that the bytes come from HBM
    NSTEP = max(1, args.steps)
    NX = min(NSTEP, 8)
    base = [make_layer(100 + r, Q4_0, Q4_0) for r in range(NX)]
    layers = step_layers(base, NSTEP, 5000, Q4_0)
    gx = torch.Generator(device=dev).manual_seed(7)
    xs = torch.randn(NSTEP, 1, H, generator=gx, device=dev)
    outs = torch.empty(NSTEP, 1, H, device=dev)
    from chimere_amd._lib import lib
    import ctypes as C

    def step_fn(i, stage=-1):
        L = layers[i % NSTEP]
        x, o = xs[i % NSTEP], outs[i % NSTEP]

        def f():
            lib().chimere_moe_ffn_decode_stage(C.byref(L.c), C.c_void_p(x.data_ptr()), C.c_void_p(o.data_ptr()), 1,
                                               C.c_void_p(L.workspace.data_ptr()), L.ws_bytes, stage, G._stream())
        return f

    # memory-side cache flush between timed replays: one 1 GiB device copy
    # (4x the 256 MB cache), so a replay of few steps still reads its
    # weights from HBM
    fl_src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
    fl_dst = torch.empty_like(fl_src)

    def flush():
        fl_dst.copy_(fl_src)

    # warm-up: W untimed steps, and one call per step layer (each workspace
    # then holds its step's routing plan for the per-kernel timing below)
    for i in range(args.warmup):
        step_fn(i)()
    for i in range(NSTEP):
        step_fn(i)()
    torch.cuda.synchronize()
    t_step, _ = graph_time([step_fn(i) for i in range(args.steps)], flush=flush)
    ms_per_step = t_step / args.steps * 1e3
    us_layer = ms_per_step * 1e3
    value = sel_bytes / (t_step / args.steps) / 1e9

    # eager (no graph) time per layer for reference
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step_fn(i)()
    torch.cuda.synchronize()
    us_eager = (time.perf_counter() - t0) / args.steps * 1e6

    # per-kernel timing: a graph of one stage's launch for every step layer
    # (plans prepared above), flushed like the headline: the kernel's average
    # launch duration under the headline's conditions
    per_kernel = {}
    NBF = F // 32
    kbytes = {
        # router weights + x + logits + Q8_1(x)
        "k_moe_route": E * H * 4 + H * 4 + E * 4 + (H // 32) * 36,
        # 9 experts' (8 routed + shared) gate/up rows + logits + Q8_1(x) + Q8_1(h) written
        "k_moe_expert1": 9 * 2 * F * row_bytes(Q4_0, H) + E * 4 + (H // 32) * 36 + 9 * NBF * 36,
        # 9 experts' down matrices + Q8_1(h) + routing weights + output
        "k_moe_dc1": 9 * H * row_bytes(Q4_0, F) + 9 * NBF * 36 + K * 4 + H * 4,
    }
    for stage, name in enumerate(["k_moe_route", "k_moe_expert1", "k_moe_dc1"]):
        n = NSTEP
        t, _ = graph_time([step_fn(i, stage) for i in range(n)], flush=flush)
        avg = t / n
        per_kernel[name] = {"us": round(avg * 1e6, 3), "alg_bytes": kbytes[name],
                            "GBs": round(kbytes[name] / avg / 1e9, 1)}
    dom = max(per_kernel, key=lambda k: per_kernel[k]["us"])
    ach = per_kernel[dom]["GBs"]
    # HBM traffic per launch of the dominant kernel, measured by the rocprofv3
    # FETCH_SIZE / WRITE_SIZE passes summarised in profiles/ (bench.py cannot
    # read hardware counters itself); null when no summary covers the kernel
    traffic, traffic_src = None, None
    tpath = os.path.join(ROOT, "profiles", "k_moe_expert1_m1_q4_0_traffic.json")
    if os.path.exists(tpath):
        tj = json.load(open(tpath))
        for kname, kv in tj["kernels"].items():
            if kname.split("::")[-1].startswith(dom):
                traffic = int(kv["read_bytes"] + kv["write_bytes"])
                traffic_src = tj["source"]
    roofline = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "kernel": dom, "alg_bytes_per_launch": kbytes[dom], "avg_launch_us": per_kernel[dom]["us"],
                "avg_launch_source": "HIP events around a graph of one launch of the kernel per step layer, "
                                     "cache flushed before each replay (the headline's conditions)"}

    extra = {"us_per_layer_m1": round(us_layer, 3), "us_per_layer_m1_eager": round(us_eager, 2),
             "GBs_selected_m1": round(value, 1), "GBs_all_bytes_m1": round(all_bytes / (t_step / args.steps) / 1e9, 1),
             "frac_of_peak_selected_m1": round(value / HBM_PEAK_GBS, 4), "per_kernel_m1": per_kernel,
             "per_kernel_timing": "graph of one launch of the kernel per step layer, cache flushed before each replay"}

    # host copies of one instance of each config and the GPU's outputs on it,
    # for the CPU baseline leg at the end (which times the reference's CPU
    # path structure on the same weights and checks it against the GPU)
    cpu_in = {}
    h = lambda t: t.detach().cpu().numpy()  # noqa: E731
    if not args.no_cpu:
        L0 = layers[0]
        o3 = L0.forward(xs[0])
        cpu_in["c3"] = ([h(t) for t in L0.tensors[:4]], tuple(h(t) for t in L0.tensors[6:9]), h(xs[0]), h(o3), Q4_0,
                        Q4_0)

    if not args.no_extra:
        # ---------------- config 4: M=8, IQ3_S experts + Q8_0 shared, uniform and Zipf routing
        rng = np.random.default_rng(5)
        perm = rng.permutation(E)
        p = np.arange(1, E + 1, dtype=np.float64) ** -1.1
        p /= p.sum()
        b = np.empty(E, np.float32)
        b[perm] = np.log(p).astype(np.float32)
        zbias = torch.from_numpy(b).to(dev)
        for label, bias in (("uniform", None), ("zipf1.1", zbias)):
            R8 = 3
            l8base = [make_layer(200 + r, IQ3_S, Q8_0, bias=bias) for r in range(R8)]
            l8 = step_layers(l8base, 96, 7000, Q8_0, bias=bias)
            x8 = torch.randn(32, 8, H, generator=gx, device=dev)
            o8 = torch.empty(8, H, device=dev)
            ids = torch.empty(8, K, dtype=torch.int32, device=dev)
            uniq = []
            for i in range(32):
                l8[i].forward(x8[i], out=o8, ids=ids, wts=torch.empty(8, K, device=dev))
                uniq.append(len(set(ids.cpu().numpy().reshape(-1).tolist())))
            if bias is None and not args.no_cpu:
                o8c = l8[0].forward(x8[0])
                cpu_in["c4"] = ([h(t) for t in l8[0].tensors[:4]], tuple(h(t) for t in l8[0].tensors[6:9]), h(x8[0]),
                                h(o8c), IQ3_S, Q8_0)
            fns = [(lambda i=i: l8[i].forward(x8[i % 32], out=o8)) for i in range(96)]
            t8, _ = graph_time(fns, flush=flush)
            us8 = t8 / 96 * 1e6
            ub = np.mean(uniq) * (2 * F * row_bytes(IQ3_S, H) + H * row_bytes(IQ3_S, F))
            extra[f"m8_iq3s_{label}"] = {"us_per_layer": round(us8, 2), "mean_unique_experts": round(float(np.mean(uniq)), 2),
                                         "GBs_unique_expert_bytes": round(ub / (us8 * 1e-6) / 1e9, 1)}
            if bias is None:
                # one token through the same IQ3_S layers, and with the reference
                # model's Q5_K shared expert (valid random Q5_K blocks: random
                # quant and scale bytes, f16 d = 1e-3, dmin = 2e-4)
                gq = torch.Generator(device=dev).manual_seed(9)

                def rand_q5k(rows, cols):
                    blk = torch.randint(0, 256, (rows, cols // 256, 176), dtype=torch.uint8, device=dev, generator=gq)
                    blk[:, :, 0:2] = torch.full((rows, cols // 256, 1), 1e-3, dtype=torch.float16,
                                                device=dev).view(torch.uint8)
                    blk[:, :, 2:4] = torch.full((rows, cols // 256, 1), 2e-4, dtype=torch.float16,
                                                device=dev).view(torch.uint8)
                    return blk.reshape(-1)
                l5 = step_layers(l8base, 96, 9000, 13,
                                 shared=lambda i, g: (rand_q5k(F, H), rand_q5k(F, H), rand_q5k(H, F)))
                x1 = torch.randn(64, 1, H, generator=gx, device=dev)
                o1 = torch.empty(1, H, device=dev)
                sel3 = K * (2 * F * row_bytes(IQ3_S, H) + H * row_bytes(IQ3_S, F))
                for tag, ls in (("m1_iq3s_q8_0", l8), ("m1_iq3s_q5k", l5)):
                    fns = [(lambda i=i, ls=ls: ls[i].forward(x1[i % 64], out=o1)) for i in range(96)]
                    t1m, _ = graph_time(fns, flush=flush)
                    u1 = t1m / 96 * 1e6
                    extra[tag] = {"us_per_layer": round(u1, 2), "GBs_selected": round(sel3 / (u1 * 1e-6) / 1e9, 1)}
                # the reference's f32-activation IQ3_S expert path (fused_moe_iq3s) on the same
                # routed experts: K experts per call, a new expert set per step, cache flushed
                from chimere_amd.moe import fused_moe_iq3s
                gf = torch.Generator(device=dev).manual_seed(11)
                fm_ids = [torch.randperm(E, generator=gf, device=dev)[:K].to(torch.int32) for _ in range(96)]
                fm_w = torch.rand(K, generator=gf, device=dev) * 0.2
                fm_out = torch.zeros(H, device=dev)
                fm_ws = torch.empty(K * F * 4, dtype=torch.uint8, device=dev)
                fm_t = [lb.tensors[1:4] for lb in l8base]
                fns = [(lambda i=i: fused_moe_iq3s(x1[i % 64, 0], *fm_t[i % len(fm_t)], fm_ids[i], fm_w, fm_out, H, F,
                                                   fm_t[0][0].shape[1], fm_t[0][1].shape[1], fm_t[0][2].shape[1], K,
                                                   workspace=fm_ws)) for i in range(96)]
                tfm, _ = graph_time(fns, flush=flush)
                ufm = tfm / 96 * 1e6
                extra["fused_moe_iq3s_f32_top8"] = {"us": round(ufm, 2), "GBs_selected": round(sel3 / (ufm * 1e-6) / 1e9, 1),
                                                    "note": "routed experts only (no router, no shared expert), f32 activations"}
                if not args.no_ncmoe:
                    # the same layer with its routed experts on the host (the
                    # reference's ncmoe path): device router + top-k, host expert
                    # loop (libchimere_cpu.so), device shared expert; one token
                    # per call, wall clock, experts rotated over the inputs
                    from chimere_amd import cpu as CPU
                    ln = l5[0]
                    ln.attach_cpu_experts(*(t.cpu().numpy() for t in ln.tensors[1:4]))
                    nc = {}
                    for nt in (4, min(16, os.cpu_count() or 1)):
                        ln.forward_ncmoe(x1[0, 0], nthreads=nt)
                        torch.cuda.synchronize()
                        ts = []
                        for i in range(24):
                            t0 = time.perf_counter()
                            ln.forward_ncmoe(x1[i % 64, 0], nthreads=nt)
                            torch.cuda.synchronize()
                            ts.append(time.perf_counter() - t0)
                        g_, u_, d_ = ln.cpu_experts
                        ids_h = np.arange(K, dtype=np.int32) * 7 % E
                        w_h = np.full(K, 1.0 / K, np.float32)
                        xh_ = x1[0, 0].cpu().numpy()
                        te = []
                        for i in range(24):
                            t0 = time.perf_counter()
                            CPU.ncmoe_experts(g_, u_, d_, (ids_h + 11 * i) % E, w_h, xh_, H, F, nthreads=nt)
                            te.append(time.perf_counter() - t0)
                        nc[f"threads_{nt}"] = {"us_per_token": round(float(np.median(ts)) * 1e6, 1),
                                               "us_cpu_experts": round(float(np.median(te)) * 1e6, 1),
                                               "GBs_cpu_selected": round(sel3 / float(np.median(te)) / 1e9, 2)}
                    nc["isa"] = ["portable", "avx2", "avx512"][CPU.lib().chimere_cpu_isa()]
                    extra["ncmoe_m1_iq3s_q5k"] = nc
                    del ln.cpu_experts
                del l5
            del l8
            torch.cuda.empty_cache()

        # ---------------- config 5: 512-token prefill chunk, Q4_0, two layer copies rotated
        T = 512
        lp = [make_layer(300 + r, Q4_0, Q4_0) for r in range(2)]
        xp = torch.randn(T, H, generator=gx, device=dev)
        op = torch.empty(T, H, device=dev)
        ids = torch.empty(T, K, dtype=torch.int32, device=dev)
        for lyr in lp:
            lyr.prefill(xp, out=op, ids=ids, wts=torch.empty(T, K, device=dev))
        ue = len(set(ids.cpu().numpy().reshape(-1).tolist()))
        if not args.no_cpu:
            cpu_in["c5"] = ([h(t) for t in lp[1].tensors[:4]], tuple(h(t) for t in lp[1].tensors[6:9]), h(xp[:16]),
                            h(op[:16]), Q4_0, Q4_0)
        fns = [(lambda i=i: lp[i % 2].prefill(xp, out=op)) for i in range(16)]
        tp, _ = graph_time(fns)
        upf = tp / 16
        pairs = T * K + T                                   # routed pairs + shared expert rows
        ops = pairs * 2 * (2 * F * H + H * F)               # int8 MACs x2 of gate, up, down
        pbytes = (ue + 1) * expert_bytes + E * H * 4 + 2 * T * H * 4
        extra["prefill_q4_0_512"] = {
            "us_per_chunk": round(upf * 1e6, 2), "tokens_per_s": round(T / upf, 1), "unique_experts": ue,
            "GBs_unique_weight_bytes": round(pbytes / upf / 1e9, 1),
            "int8_TOPs": round(ops / upf / 1e12, 2), "mfma_frac_of_int8_peak": round(ops / upf / 1e12 / 5000.0, 4)}
        del lp
        torch.cuda.empty_cache()

        # the same chunk with IQ3_S experts (the reference model's quantization),
        # IQ3_S or Q8_0 shared expert
        for tag, st in (("prefill_iq3s_512", IQ3_S), ("prefill_iq3s_q8_0_shared_512", Q8_0)):
            lp = [make_layer(310 + r, IQ3_S, st) for r in range(2)]
            for lyr in lp:
                lyr.prefill(xp, out=op, ids=ids, wts=torch.empty(T, K, device=dev))
            ue = len(set(ids.cpu().numpy().reshape(-1).tolist()))
            fns = [(lambda i=i: lp[i % 2].prefill(xp, out=op)) for i in range(16)]
            tp, _ = graph_time(fns)
            upf = tp / 16
            eb = 2 * F * row_bytes(IQ3_S, H) + H * row_bytes(IQ3_S, F)
            sb = 2 * F * row_bytes(st, H) + H * row_bytes(st, F)
            pbytes = ue * eb + sb + E * H * 4 + 2 * T * H * 4
            extra[tag] = {"us_per_chunk": round(upf * 1e6, 2), "tokens_per_s": round(T / upf, 1),
                          "unique_experts": ue, "GBs_unique_weight_bytes": round(pbytes / upf / 1e9, 1),
                          "int8_TOPs": round(ops / upf / 1e12, 2)}
            del lp
            torch.cuda.empty_cache()

        # ---------------- config 2: Q4_0 head 151936 x 2048, three copies rotated
        V = 151936
        g = torch.Generator(device=dev).manual_seed(2)
        heads = [qmat(Q4_0, V, H, 1, g)[0] for _ in range(3)]
        xq = torch.empty(G.q8_1_row_bytes(H), dtype=torch.uint8, device=dev)
        G.ggml_gpu_quantize_q8_1(torch.randn(H, generator=g, device=dev), xq, H)
        y = torch.empty(V, device=dev)
        fns = [(lambda i=i: G.ggml_gpu_gemv_q4_0_q8(heads[i % 3], xq, y, V, H)) for i in range(30)]
        th, _ = graph_time(fns)
        hb = V * row_bytes(Q4_0, H) + V * 4 + (H // 32) * 36
        extra["head_q4_0_151936x2048"] = {"us": round(th / 30 * 1e6, 2), "GBs": round(hb / (th / 30) / 1e9, 1),
                                          "frac": round(hb / (th / 30) / 1e9 / HBM_PEAK_GBS, 4)}
        if not args.no_cpu:
            G.ggml_gpu_gemv_q4_0_q8(heads[0], xq, y, V, H)
            cpu_in["c2"] = (h(heads[0]), h(xq), h(y), Q4_0, V)
        del heads
        # ---------------- config 1: Q8_0 4096 x 2048, 64 copies rotated (570 MB)
        q8w = qmat(Q8_0, 4096, H, 64, g)
        y1 = torch.empty(4096, device=dev)
        fns = [(lambda i=i: G.ggml_gpu_gemv_q8_0_q8(q8w[i % 64], xq, y1, 4096, H)) for i in range(256)]
        t1, _ = graph_time(fns)
        b1 = 4096 * row_bytes(Q8_0, H) + 4096 * 4 + (H // 32) * 36
        extra["dense_q8_0_4096x2048"] = {"us": round(t1 / 256 * 1e6, 2), "GBs": round(b1 / (t1 / 256) / 1e9, 1)}
        if not args.no_cpu:
            G.ggml_gpu_gemv_q8_0_q8(q8w[0], xq, y1, 4096, H)
            cpu_in["c1"] = (h(q8w[0]), h(xq), h(y1), Q8_0, 4096)
        del q8w
        # ---------------- ggml K-quant / MXFP4 GEMV, 16384 x 4096, four copies rotated (timing
        # only: random block bytes)
        Rk, Ck = 16384, 4096
        xk = torch.empty(G.q8_1_row_bytes(Ck), dtype=torch.uint8, device=dev)
        G.ggml_gpu_quantize_q8_1(torch.randn(Ck, generator=g, device=dev), xk, Ck)
        yk = torch.empty(Rk, device=dev)
        for name, fn, rbk in (("q4k", G.ggml_gpu_gemv_q4k_q8, Ck // 256 * 144), ("q5k", G.ggml_gpu_gemv_q5k_q8, Ck // 256 * 176),
                              ("q6k", G.ggml_gpu_gemv_q6k_q8, Ck // 256 * 210), ("mxfp4", G.ggml_gpu_gemv_mxfp4_q8, Ck // 32 * 17)):
            wk = torch.randint(0, 256, (4, Rk * rbk), dtype=torch.uint8, device=dev, generator=g)
            fns = [(lambda i=i, fn=fn, wk=wk: fn(wk[i % 4], xk, yk, Rk, Ck)) for i in range(32)]
            tk, _ = graph_time(fns)
            bk = Rk * rbk + Rk * 4 + (Ck // 32) * 36
            extra[f"{name}_{Rk}x{Ck}"] = {"us": round(tk / 32 * 1e6, 2), "GBs": round(bk / (tk / 32) / 1e9, 1),
                                          "frac": round(bk / (tk / 32) / 1e9 / HBM_PEAK_GBS, 4)}
            del wk

        # ---------------- attainable rates on this part (beside the datasheet peaks)
        import ctypes as _C
        _probe = _C.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "chimere_amd", "libchimere_probe.so"))
        _probe.chimere_probe_stream_read.argtypes = [_C.c_void_p, _C.c_int64, _C.c_void_p, _C.c_int, _C.c_void_p]
        _probe.chimere_probe_mfma_i8.argtypes = [_C.c_void_p, _C.c_int, _C.c_int, _C.c_void_p]
        _clib = lambda: _probe  # noqa: E731
        big = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
        big.fill_(1)
        fold = torch.empty(8192, dtype=torch.int32, device=dev)
        best_rd = 0.0
        for nb in (1024, 2048, 4096, 8192):
            fns = [(lambda nb=nb: _clib().chimere_probe_stream_read(_C.c_void_p(big.data_ptr()), big.numel(),
                                                                  _C.c_void_p(fold.data_ptr()), nb, G._stream()))
                   for _ in range(3)]
            tr, _ = graph_time(fns)
            best_rd = max(best_rd, big.numel() / (tr / 3) / 1e9)
        del big
        mo = torch.empty(1024 * 256, dtype=torch.int32, device=dev)
        iters = 4000
        fns = [lambda: _clib().chimere_probe_mfma_i8(_C.c_void_p(mo.data_ptr()), iters, 1024, G._stream())]
        tm, _ = graph_time(fns)
        mops = 1024 * 4 * 4 * iters * 2 * 32 * 32 * 32 / tm / 1e12
        extra["attainable"] = {"hbm_read_GBs": round(best_rd, 1), "hbm_read_frac_of_peak": round(best_rd / HBM_PEAK_GBS, 4),
                               "mfma_i8_TOPs": round(mops, 1), "mfma_i8_frac_of_peak": round(mops / 5000.0, 4),
                               "method": "2 GiB non-temporal dwordx4 read, best of 1024-8192 work-groups; "
                                         "1024 WGs x 4 waves x 4 chains of v_mfma_i32_32x32x32_i8"}

    # ---------------- CPU baseline: the reference's CPU path structure
    # (oracle/cpu_path.c: Q8_1 activations once per call, OpenMP row-parallel
    # AVX2 vec_dots, cs/ffi/ggml_iq3s_gemv.c:84-127) on this host, for each
    # config, with all host threads of this GPU's share and with one thread;
    # each figure is the median call time over a bounded sample
    cpu = None
    if not args.no_cpu:
        import oracle as O
        nthr = min(16, os.cpu_count() or 1)

        def ctime(fn, budget=args.cpu_seconds / 10):
            fn()
            ts, t_end = [], time.perf_counter() + budget
            while len(ts) < 3 or (time.perf_counter() < t_end and len(ts) < 200):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
            return float(np.median(ts)), len(ts)

        def rel(a, b):
            return float(np.linalg.norm(np.ravel(a) - np.ravel(b)) / max(np.linalg.norm(np.ravel(b)), 1e-30))

        configs = {}
        for key, name in (("c1", "config1_dense_q8_0_4096x2048"), ("c2", "config2_head_q4_0_151936x2048")):
            if key not in cpu_in:
                continue
            W, xqh, yg, t, nrows = cpu_in[key]
            rec = {}
            for tag, n in (("threads", nthr), ("single_thread", 1)):
                dt, calls = ctime(lambda: O.cpu_gemv(t, W, xqh, H, nrows, nthreads=n))
                rec[tag] = {"n": n, "us": round(dt * 1e6, 1),
                            "GBs": round((W.size + nrows * 4 + xqh.size) / dt / 1e9, 2), "calls": calls}
            rec["rel_err_vs_gpu"] = rel(O.cpu_gemv(t, W, xqh, H, nrows, nthreads=nthr), yg)
            configs[name] = rec
        for key, name, M in (("c3", "config3_moe_m1_q4_0", 1), ("c4", "config4_moe_m8_iq3s_uniform", 8),
                             ("c5", "config5_prefill_q4_0_sample16", 16)):
            if key not in cpu_in:
                continue
            (r_, gt, ut, dt_), sh, xh, og, et, st = cpu_in[key]
            xh = xh.reshape(-1, H)[:M]
            run = lambda n: O.cpu_moe(xh, r_, gt, ut, dt_, et, K, sh=sh, sh_type=st, nthreads=n)  # noqa: E731
            rec = {"tokens": M}
            for tag, n in (("threads", nthr), ("single_thread", 1)):
                dtm, calls = ctime(lambda: run(n))
                ent = {"n": n, "us_per_call": round(dtm * 1e6, 1), "calls": calls}
                if key == "c3":
                    ent["GBs_selected"] = round(sel_bytes / dtm / 1e9, 3)
                else:
                    ent["tokens_per_s"] = round(M / dtm, 1)
                rec[tag] = ent
            oc, _, _ = run(nthr)
            errs = [rel(oc[m], og.reshape(-1, H)[m]) for m in range(M)]
            rec["rel_err_vs_gpu"] = max(errs)
            rec["rel_err_vs_gpu_median"] = float(np.median(errs))
            if key == "c4":
                oo, _, _ = O.moe(xh, r_, gt, ut, dt_, et, K, sh=sh, sh_type=st, nthreads=nthr)
                rec["rel_err_oracle_vs_gpu"] = max(rel(oo[m], og.reshape(-1, H)[m]) for m in range(M))
                rec["note"] = ("CPU path in its own fp32 order vs GPU (L=16 order): a one-ulp gate/up difference "
                               "can move one Q8_1(h) rounding step; oracle in the GPU's order vs GPU: bit-exact")
            if key == "c5":
                # the CPU path sums in its own (AVX2) fp32 order and the GPU
                # prefill in the L=1 order: a one-ulp difference in a gate/up
                # value can move one Q8_1(h) rounding step, worth ~1e-5 of the
                # output.  The same tokens through the oracle in the prefill's
                # order give the GPU's bits.
                oo, _, _ = O.moe(xh, r_, gt, ut, dt_, et, K, sh=sh, sh_type=st, L=1, nthreads=nthr)
                rec["rel_err_oracle_prefill_order_vs_gpu"] = max(rel(oo[m], og.reshape(-1, H)[m]) for m in range(M))
                rec["note"] = ("CPU path in its own fp32 order vs GPU prefill (L=1 order): one Q8_1(h) rounding "
                               "step moved on some tokens; oracle in the prefill order vs GPU: bit-exact")
            configs[name] = rec
        c3 = configs.get("config3_moe_m1_q4_0")
        model = ""
        try:
            for ln in open("/proc/cpuinfo"):
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
        cpu = {"value": c3["threads"]["GBs_selected"], "unit": "GB/s", "cores": nthr, "kind": "port",
               "sample": f"config 3 (M=1 Q4_0 MoE layer) on the CPU path restatement oracle/cpu_path.c "
                         f"({c3['threads']['calls']} calls, median {c3['threads']['us_per_call']} us/layer); "
                         f"configs 1-5 in 'configs' (config 5: 16 tokens of the 512-token chunk, one token at a "
                         f"time as the reference's prefill does)",
               "single_thread_GBs": c3["single_thread"]["GBs_selected"], "nproc": os.cpu_count(),
               "cpu_model": model, "configs": configs}

    if args.calib_copy_mb:
        src = torch.empty(args.calib_copy_mb << 18, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        extra["calib_copy_bytes_each_way"] = args.calib_copy_mb << 20

    line = {"metric": "MoE decode FFN effective HBM GB/s on selected-expert bytes (M=1, Q4_0, Qwen3.5-35B-A3B shape)",
            "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8", "data": "synthetic",
            "config": {"workload": "BASELINE config 3: MoE decode FFN layer M=1 Q4_0, H=2048 F=512 E=256 top-8 + shared",
                       "hidden": H, "ffn": F, "experts": E, "top_k": K, "tokens": 1,
                       "step_layers": NSTEP, "routed_expert_copies": NX,
                       "timing": "median of 5 graph replays of exactly `steps` layer calls, each step its own "
                                 "router, shared expert and token (routed experts from one of up to 8 copies); a "
                                 "1 GiB device copy (4x the memory-side cache) runs untimed before each replay"},
            "roofline": roofline, "cpu_baseline": cpu, "extra": extra}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
