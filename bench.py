#!/usr/bin/env python3
"""Benchmark of the MI355X MoE block (BASELINE.json metric).

Headline (`value`): decode tokens/s at B=1 through the 40-layer MoE-only stack
each step is one token through 40 layers of
x_{l+1} = x_l + MoE_l(RMSNorm(x_l)), all 40 x 256 experts resident in one
HBM arena, inputs resident in HBM before timing.  Also reported:
  * hbm_gbs: algorithmic bytes/token (40 x 19,619,840 B) x tokens/s;
  * prefill512_tflops: BASELINE config 3 (512 tokens, one layer, Zipf s=1
    router bias), 29.53 GFLOP per call / time, with its roofline (AI x HBM
    peak vs the fp16 MFMA peak) and the routed grouped-GEMM rate alone;
  * prefill8192_zipf13: BASELINE config 4 (8192 tokens, one layer, Zipf s=1.3),
    472.5 GFLOP per call / time;
  * cfg0_decode_b1_layer: BASELINE config 0, one layer, B=1, calls rotated
    over the 40 resident layers (so the 256 MB MALL holds none of them);
  * cfg1_decode_b8_zipf_layer: BASELINE config 1, one layer, B=8 with the
    Zipf s=1 router bias, rotated over the 40 layers; bytes count each distinct
    expert of a call once (the reference's accounting);
  * stack40_b8: 8 tokens per step through the 40-layer stack (no bias);
  * convert_layer_q8_0: the IQ4_NL converter, one layer's routed experts
    (blk.N.ffn_{gate,up,down}_exps in Q8_0, the reference converter's input)
    quantized into the arena, against the CPU restatement of ggml's quantizer
    on a few experts (--convert-only runs just this, for profiling);
  * roofline: the decode kernel (k_decode, the only kernel of a decode step:
    one launch per step), its duration the timed region's HIP-event time per
    step on the launch stream;
  * cpu_baseline: the CPU AVX2 restatement of the reference CPU MoE path
    (oracle/qe_oracle.cpp) on a bounded sample, host cores, same process, at
    the box's thread share and at the reference's default of 12 threads; the
    prefill lines carry their own CPU baseline (GFLOP/s of the same layer).
Weights are random-init from the seeded generator (no checkpoints offline).
"""
import argparse
import ctypes
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "qe-qwen36-b50_amd"))

import numpy as np  # noqa: E402

METRIC = "MoE decode tokens/s + HBM GB/s at B=1; prefill-512 MoE TFLOPS (1 GPU)"
EXPERT_BYTES = 1769472
LAYER_BYTES_B1 = 8 * EXPERT_BYTES + 1024 * 2176 + 2048 * 544 + 257 * 2048 * 4 + 2 * 8192  # 19,619,840
N_LAYERS = 40
FLOP_PER_TOKEN = 8 * 6291456 + 6291456 + 2 * 257 * 2048  # 57,675,776
HBM_PEAK = 8.0e12
FP16_PEAK = 2.5e15
INT8_PEAK = 5.0e15
DENSE_BYTES = 1024 * 2176 + 2048 * 544 + 257 * 2048 * 4 + 2048 * 4  # shared Q8, router, post_norm
ROUTED_FLOP_PER_PAIR = 2 * 1024 * 2048 + 2 * 2048 * 512  # gate/up + down of one (token, expert) pair
SEED = 0x51E3_6B50
TRAFFIC_FILE = "profiles/k_decode_cfg2_pmc.txt"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def timed(torch, fn, steps, stream):
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        fn()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def layer_rotation(torch, m, x, y, T, n_layers, steps):
    """One-layer calls (forward_normed: no norm, no residual) cycling over
    n_layers resident layers, HIP events on the launch stream; ms per call."""
    st = torch.cuda.current_stream()
    i = [0]

    def call():
        m.forward_normed(i[0] % n_layers, x, y, T, stream=st)
        i[0] += 1

    for _ in range(n_layers):
        call()
    return timed(torch, call, steps, st)


def cpu_prefill(T, inst, bias_s, threads, budget_s):
    """The reference's batched CPU expert path (engine/qe.cpp:2050-2101, restated
    in oracle/qe_oracle.cpp as orc_baseline_layer) over one whole prefill layer:
    router, top-8, dispatch, int8 experts, Q8 shared expert, combine; the same
    seeded layer (all 256 experts) and input as the GPU line.  Runs until
    budget_s of timed work (at least once).  Returns (GFLOP/s, ms per call, calls)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    import qe_moe

    L = O.SynthLayer(SEED, 0, bias=qe_moe.synth_zipf_bias(SEED, 0, bias_s))
    blobs = [O.gen_expert(SEED, 0, e) for e in range(256)]
    ptrs = (ctypes.c_void_p * 256)()
    for e, b in enumerate(blobs):
        ptrs[e] = b.ctypes.data
    x = O.gen_x(SEED, inst, T)
    total, calls = 0.0, 0
    while calls == 0 or total < budget_s:
        sec, _ = O.baseline_layer(x, None, L, ptrs, T, threads)
        total += sec
        calls += 1
    return T * FLOP_PER_TOKEN / (total / calls) / 1e9, total / calls * 1e3, calls


def cpu_baseline(n_distinct, budget_s, max_tokens, threads):
    """The reference CPU MoE path (the AVX2 restatement in oracle/qe_oracle.cpp,
    full layer: norm, router, top-8, dispatch, int8 experts, Q8 shared expert,
    combine, residual) decoding B=1 tokens through the 40-layer stack on host
    cores.  Bounded sample: n_distinct synthetic layers (all 256 experts each)
    are cycled to form the 40 layer steps, and tokens run until budget_s of
    timed CPU work (or max_tokens).  Returns (tokens/s, seconds, tokens)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    layers, ptr_sets, blobs = [], [], []
    for l in range(n_distinct):
        L = O.SynthLayer(SEED + 7, l)
        ptrs = (ctypes.c_void_p * 256)()
        for e in range(256):
            b = O.gen_expert(SEED + 7, l, e)
            blobs.append(b)
            ptrs[e] = b.ctypes.data
        layers.append(L)
        ptr_sets.append(ptrs)
    pn = np.ones(2048, np.float32)
    total, tokens = 0.0, 0
    while tokens < max_tokens and (total < budget_s or tokens == 0):
        h = O.gen_x(SEED + 7, 1000 + tokens, 1)
        for step in range(N_LAYERS):
            li = step % n_distinct
            sec, h = O.baseline_layer(h, pn, layers[li], ptr_sets[li], 1, threads)
            total += sec
        tokens += 1
    return tokens / total, total, tokens


CONVERT_SRC_BYTES = 3 * 256 * 1048576 // 32 * 34  # Q8_0 gate, up, down of one layer
CONVERT_DST_BYTES = 256 * EXPERT_BYTES


def convert_bench(torch, qe_moe, steps, cpu_experts, threads):
    """One layer of Q8_0 experts -> arena blobs (qe_moe_convert_experts), HIP events on the launch stream."""
    g = torch.Generator(device="cuda")
    g.manual_seed(SEED)

    def q8(nblk):
        t = torch.randint(0, 256, (nblk, 34), dtype=torch.uint8, device="cuda", generator=g)
        t[:, :2] = (torch.rand(nblk, device="cuda", generator=g) * 0.02).half().view(torch.uint8).view(nblk, 2)
        return t

    gate, up, down = q8(256 * 512 * 64), q8(256 * 512 * 64), q8(256 * 2048 * 16)
    m = qe_moe.MoE(n_layers=1, t_max=16)
    st = torch.cuda.current_stream()
    run = lambda: m.convert_experts(0, gate, up, down, qe_moe.SRC_Q8_0, stream=st)  # noqa: E731
    run()
    ms = timed(torch, run, steps, st)
    res = {"ms": round(ms, 4), "blocks": 3 * 256 * 1048576 // 32,
           "algorithmic_bytes": CONVERT_SRC_BYTES + CONVERT_DST_BYTES,
           "gbs": round((CONVERT_SRC_BYTES + CONVERT_DST_BYTES) / (ms / 1e3) / 1e9, 1),
           "hbm_frac": round((CONVERT_SRC_BYTES + CONVERT_DST_BYTES) / (ms / 1e3) / HBM_PEAK, 4),
           "bound": "lds (bank conflicts of the nearest-entry slot reads: 16 candidate scales x 32 elements per block)"}
    if cpu_experts:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O

        hg, hu, hd = (t.cpu().numpy() for t in (gate, up, down))
        O.load().orc_set_threads(threads)
        t0 = time.perf_counter()
        for e in range(cpu_experts):
            O.convert_expert(hg, hu, hd, O.SRC_Q8_0, e)
        cs = time.perf_counter() - t0
        res["cpu_baseline"] = {"ms_per_layer": round(cs / cpu_experts * 256 * 1e3, 1), "cores": threads, "kind": "port",
                               "sample": f"{cpu_experts} experts of the same layer, scaled to 256"}
    m.close()
    return res


def cpu_host(threads):
    """The host CPU the baseline ran on, from lscpu: model, sockets, cores per
    socket, threads per core, logical CPUs, and how many of them this process
    may use (its affinity: the box's CPU share) and used (threads)."""
    info = {}
    try:
        import subprocess

        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        kv = {l.split(":", 1)[0].strip(): l.split(":", 1)[1].strip() for l in txt.splitlines() if ":" in l}
        info = {"model": kv.get("Model name"), "sockets": kv.get("Socket(s)"), "cores_per_socket": kv.get("Core(s) per socket"),
                "threads_per_core": kv.get("Thread(s) per core"), "logical_cpus": kv.get("CPU(s)"),
                "hypervisor": kv.get("Hypervisor vendor")}
    except (OSError, ValueError):
        pass
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except OSError:
        pass
    info["threads_used"] = threads
    return info


def pmc_traffic(path):
    """HBM bytes per k_decode dispatch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE in KiB per dispatch, each divided by the factor
    the same counter reads for a plain copy of known size).  None if absent."""
    if not os.path.exists(path):
        return None
    kv = {}
    for line in open(path):
        if ":" in line and not line.startswith("#"):
            k, v = line.split(":", 1)
            try:
                kv[k.strip()] = float(v.split()[0])
            except (ValueError, IndexError):
                pass
    try:
        return (kv["fetch_kib_per_dispatch"] / kv["copy_fetch_factor"]
                + kv["write_kib_per_dispatch"] / kv["copy_write_factor"]) * 1024.0
    except KeyError:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--graph", action="store_true", help="replay a captured HIP graph (one launch per step anyway)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the decode lines (profiling the prefill kernels alone); no headline value")
    ap.add_argument("--prefill-configs", default="3,4", help="BASELINE prefill configs to run (3: 512 tokens, 4: 8192)")
    ap.add_argument("--cpu-layers", type=int, default=8, help="distinct synthetic layers cycled by the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="timed CPU work of the baseline sample")
    ap.add_argument("--cpu-threads", type=int, default=16, help="host threads of the CPU baseline (the box's CPU share)")
    ap.add_argument("--no-convert", action="store_true", help="skip the IQ4_NL converter side line")
    ap.add_argument("--convert-only", action="store_true", help="run only the converter side line (profiling)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run a plain device copy of this many bytes 5 times (PMC calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU expert sharding is design-only in this build", file=sys.stderr)
        sys.exit(2)

    import torch

    assert torch.cuda.is_available(), "no GPU visible"
    dev = torch.device("cuda:0")
    if args.copy_bytes:
        src = torch.empty(args.copy_bytes, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": args.copy_bytes, "copies": 5}))
        return

    import qe_moe

    threads = max(1, min(os.cpu_count() or 1, args.cpu_threads))
    if args.convert_only:
        print(json.dumps({"convert_layer_q8_0": convert_bench(torch, qe_moe, 5, 0, threads)}), flush=True)
        return

    stream = torch.cuda.current_stream()

    dec = None
    if not args.no_decode:
        # ---------------- config 2: 40-layer decode, B=1 ----------------
        log("building 40-layer arena (18.12 GB) from the seeded generator")
        m = qe_moe.MoE(n_layers=N_LAYERS, t_max=16)
        for l in range(N_LAYERS):
            m.synth_layer(l, SEED, None, stream=stream)
        x = torch.empty(1, 2048, device=dev)
        qe_moe.synth_x(SEED, 0, x, x.numel(), stream=stream)
        y = torch.empty_like(x)
        torch.cuda.synchronize()

        def step_eager():
            m.forward_stack(0, N_LAYERS, x, y, 1, stream=torch.cuda.current_stream())

        step_eager()
        torch.cuda.synchronize()
        y_eager = y.clone()
        step = step_eager
        graph_used = False
        if args.graph:
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                step_eager()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            with torch.cuda.graph(g):
                step_eager()
            ok = True
            for _ in range(3):  # every replay must equal the eager result
                y.zero_()
                g.replay()
                torch.cuda.synchronize()
                ok = ok and torch.equal(y, y_eager)
                step_eager()
                torch.cuda.synchronize()
            if ok:
                step, graph_used = g.replay, True
            else:
                log("graph replay differs from eager: timing eager launches")
        log(f"decode: warmup {args.warmup}, timed {args.steps} (graph={graph_used})")
        for _ in range(args.warmup):
            step()
        ms = timed(torch, step, args.steps, torch.cuda.current_stream())
        tok_s = 1000.0 / ms
        assert torch.equal(y, y_eager), "timed output differs from the eager reference"

        # one step is one k_decode launch, so the timed region's time per step is the
        # kernel's average launch duration (back-to-back launches on one stream)
        dec_avg_s = ms / 1e3
        dec_bytes = N_LAYERS * LAYER_BYTES_B1  # one launch = one token through all 40 layers
        achieved = dec_bytes / dec_avg_s
        # per-kernel HIP events (the library's profiler) over a short pass, for reference
        m.profile(True)
        for _ in range(min(args.steps, 20)):
            step_eager()
        torch.cuda.synchronize()
        prof = m.profile_read()
        m.profile(False)
        kernels = {"source": "the library's per-launch HIP event pairs (qe_moe_profile) over a separate 20-step pass, "
                             "not the timed loop: each bracketed launch pays the events' own cost; roofline.avg_us "
                             "and profiles/k_decode_cfg2_kernel_stats.txt (rocprofv3) are the kernel's duration",
                   **{k: {"avg_us": round(v[0] / v[1] * 1e3, 3), "launches": v[1]} for k, v in prof.items()}}

        # config 0: one layer, B=1, rotated over the 40 resident layers
        x1 = torch.empty(1, 2048, device=dev)
        qe_moe.synth_x(SEED, 10, x1, x1.numel(), stream=stream)
        y1 = torch.empty_like(x1)
        ms0 = layer_rotation(torch, m, x1, y1, 1, N_LAYERS, max(200, args.steps))
        cfg0 = {"us_per_call": round(ms0 * 1e3, 3), "tokens_per_s": round(1000.0 / ms0, 1),
                "algorithmic_bytes": LAYER_BYTES_B1, "gbs": round(LAYER_BYTES_B1 / (ms0 / 1e3) / 1e9, 2),
                "hbm_frac": round(LAYER_BYTES_B1 / (ms0 / 1e3) / HBM_PEAK, 4),
                "note": "one launch per call (forward_normed, k_decode over 1 layer), calls cycle over 40 layers "
                        "(18.1 GB, beyond the 256 MB MALL); includes the per-launch fixed cost"}

        # batched decode, 8 tokens per step through the same 40 layers (the T <= 8 kernel)
        x8 = torch.empty(8, 2048, device=dev)
        qe_moe.synth_x(SEED, 1, x8, x8.numel(), stream=stream)
        y8 = torch.empty_like(x8)
        step8 = lambda: m.forward_stack(0, N_LAYERS, x8, y8, 8, stream=torch.cuda.current_stream())  # noqa: E731
        for _ in range(5):
            step8()
        ms8 = timed(torch, step8, max(20, args.steps // 4), torch.cuda.current_stream())
        stack40_b8 = {"tokens_per_s": round(8000.0 / ms8, 1), "ms_per_step": round(ms8, 4),
                      "note": "8 tokens per step through the 40-layer stack, no router bias (not BASELINE config 1)"}

        # one layer per call at T = 8 (the persistent decode kernel), 9, 12 and 16
        # (the prefill launches), no bias, rotated over the 40 layers: where the
        # two plans cross (the reference switches to its GEMV rounds below 16
        # tokens, engine/qe.cpp:2008-2027)
        small_t = {}
        for T_ in (8, 9, 12, 16):
            xs_ = torch.empty(T_, 2048, device=dev)
            qe_moe.synth_x(SEED, 20 + T_, xs_, xs_.numel(), stream=stream)
            ys_ = torch.empty_like(xs_)
            u_ = []
            for l in range(N_LAYERS):
                m.forward_normed(l, xs_, ys_, T_, stream=stream)
                u_.append(int(np.count_nonzero(np.diff(m.routing(T_, stream=stream)["off"]))))
            ms_ = layer_rotation(torch, m, xs_, ys_, T_, N_LAYERS, max(100, args.steps // 2))
            small_t[str(T_)] = {"us_per_call": round(ms_ * 1e3, 3), "tokens_per_s": round(T_ * 1000.0 / ms_, 1),
                                "distinct_experts_mean": round(float(np.mean(u_)), 2),
                                "plan": "k_decode (persistent)" if T_ <= 8 else "prefill launches"}

        # config 1: one layer, B=8, Zipf s=1 router bias, rotated over the 40 layers
        for l in range(N_LAYERS):
            m.set_dense(l, bias=qe_moe.synth_zipf_bias(SEED, l, 1.0), stream=stream)
        x8b = torch.empty(8, 2048, device=dev)
        qe_moe.synth_x(SEED, 11, x8b, x8b.numel(), stream=stream)
        uniq = []
        for l in range(N_LAYERS):
            m.forward_normed(l, x8b, y8, 8, stream=stream)
            uniq.append(int(np.count_nonzero(np.diff(m.routing(8, stream=stream)["off"]))))
        ms1 = layer_rotation(torch, m, x8b, y8, 8, N_LAYERS, max(200, args.steps))
        b1 = float(np.mean(uniq)) * EXPERT_BYTES + 5447680 + 131072
        cfg1 = {"us_per_call": round(ms1 * 1e3, 3), "tokens_per_s": round(8000.0 / ms1, 1),
                "distinct_experts_mean": round(float(np.mean(uniq)), 2), "distinct_experts_min_max": [min(uniq), max(uniq)],
                "algorithmic_bytes_mean": int(b1), "gbs": round(b1 / (ms1 / 1e3) / 1e9, 2),
                "hbm_frac": round(b1 / (ms1 / 1e3) / HBM_PEAK, 4),
                "note": "bytes = U x 1,769,472 (each distinct expert once) + 5,447,680 dense + 131,072 activations; "
                        "one launch per call, calls cycle over 40 layers with per-layer Zipf(1.0) biases"}
        del m
        torch.cuda.empty_cache()
        dec = dict(tok_s=tok_s, ms=ms, graph_used=graph_used, dec_avg_s=dec_avg_s, dec_bytes=dec_bytes,
                   achieved=achieved, kernels=kernels, cfg0=cfg0, cfg1=cfg1, stack40_b8=stack40_b8, small_t=small_t)

    # ---------------- config 3: prefill 512, one layer ----------------
    pre = {}
    pcfg = set() if args.no_prefill else {c.strip() for c in args.prefill_configs.split(",")}
    if "3" in pcfg:
        bias = qe_moe.synth_zipf_bias(SEED, 0, 1.0)
        mp = qe_moe.MoE(n_layers=1, t_max=512)
        mp.synth_layer(0, SEED, bias, stream=stream)
        xp = torch.empty(512, 2048, device=dev)
        qe_moe.synth_x(SEED, 3, xp, xp.numel(), stream=stream)
        yp = torch.empty_like(xp)
        for _ in range(3):
            mp.forward_normed(0, xp, yp, 512, stream=torch.cuda.current_stream())
        pms = timed(torch, lambda: mp.forward_normed(0, xp, yp, 512, stream=torch.cuda.current_stream()),
                    max(5, args.steps // 10), torch.cuda.current_stream())
        mp.profile(True)
        for _ in range(5):
            mp.forward_normed(0, xp, yp, 512, stream=torch.cuda.current_stream())
        torch.cuda.synchronize()
        pk = mp.profile_read()
        mp.profile(False)
        r = mp.routing(512)
        cnt = np.diff(r["off"])
        flop = 512 * FLOP_PER_TOKEN
        pbytes = int(np.count_nonzero(cnt)) * EXPERT_BYTES + DENSE_BYTES + 2 * 512 * 2048 * 4
        ai = flop / pbytes
        ceiling = min(FP16_PEAK, ai * HBM_PEAK)
        achieved_p = flop / (pms / 1e3)
        gkey = [k for k in pk if k.startswith("k_expert_gu")][0]
        g_s = pk[gkey][0] / pk[gkey][1] / 1e3
        routed_flop = 512 * 8 * ROUTED_FLOP_PER_PAIR
        pre = {"prefill512_ms": round(pms, 4), "prefill512_tflops": round(achieved_p / 1e12, 3),
               "prefill512_roofline": {"bound": "hbm" if ai * HBM_PEAK < FP16_PEAK else "mfma",
                                       "algorithmic_bytes": pbytes, "flop": flop, "ai_flop_per_byte": round(ai, 1),
                                       "ceiling_tflops": round(ceiling / 1e12, 1),
                                       "frac": round(achieved_p / ceiling, 4)},
               "prefill512_routed_gemm": {"kernels": gkey, "us": round(g_s * 1e6, 2), "flop": routed_flop,
                                          "tops": round(routed_flop / g_s / 1e12, 2), "mfma": "i32_16x16x32_i8",
                                          "frac_int8_peak": round(routed_flop / g_s / INT8_PEAK, 4),
                                          "frac_fp16_peak": round(routed_flop / g_s / FP16_PEAK, 4),
                                          "note": "time includes the shared-expert down tiles (1.07 GFLOP) of the same launch",
                                          "source": "per-launch HIP event pairs of the library profiler over 5 calls after "
                                                    "the timed loop (rocprofv3 durations: profiles/prefill512_zipf1_kernel_stats.txt)"},
               "prefill512_routing": {"distinct_experts": int(np.count_nonzero(cnt)), "max_tokens_per_expert": int(cnt.max()),
                                      "top8_share": round(float(np.sort(cnt)[-8:].sum() / cnt.sum()), 4),
                                      "experts_lt4_tokens": int(((cnt > 0) & (cnt < 4)).sum())},
               "prefill512_kernels_us": {"source": "per-launch HIP event pairs of the library profiler, 5 calls",
                                         **{k: round(v[0] / v[1] * 1e3, 2) for k, v in pk.items()}}}
        del mp, xp, yp
        torch.cuda.empty_cache()

    if "4" in pcfg:
        # config 4: prefill 8192, one layer, Zipf s=1.3 router bias
        T4 = 8192
        m4 = qe_moe.MoE(n_layers=1, t_max=T4)
        m4.synth_layer(0, SEED, qe_moe.synth_zipf_bias(SEED, 0, 1.3), stream=stream)
        x4 = torch.empty(T4, 2048, device=dev)
        qe_moe.synth_x(SEED, 4, x4, x4.numel(), stream=stream)
        y4 = torch.empty_like(x4)
        for _ in range(2):
            m4.forward_normed(0, x4, y4, T4, stream=torch.cuda.current_stream())
        ms4 = timed(torch, lambda: m4.forward_normed(0, x4, y4, T4, stream=torch.cuda.current_stream()),
                    max(3, args.steps // 40), torch.cuda.current_stream())
        c4 = np.diff(m4.routing(T4)["off"])
        f4 = T4 * FLOP_PER_TOKEN
        pre["prefill8192_zipf13"] = {"ms": round(ms4, 4), "tflops": round(f4 / (ms4 / 1e3) / 1e12, 2),
                                     "frac_fp16_peak": round(f4 / (ms4 / 1e3) / FP16_PEAK, 4),
                                     "distinct_experts": int(np.count_nonzero(c4)), "max_tokens_per_expert": int(c4.max()),
                                     "top8_share": round(float(np.sort(c4)[-8:].sum() / c4.sum()), 4),
                                     "experts_lt4_tokens": int(((c4 > 0) & (c4 < 4)).sum())}
        del m4, x4, y4
        torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        for key, T_, inst, s_ in (("prefill512", 512, 3, 1.0), ("prefill8192_zipf13", 8192, 4, 1.3)):
            if (key == "prefill512" and "3" not in pcfg) or (key != "prefill512" and "4" not in pcfg):
                continue
            log(f"cpu baseline: {key}")
            gf, cms, ncall = cpu_prefill(T_, inst, s_, threads, args.cpu_seconds / 2)
            entry = {"value": round(gf, 2), "unit": "GFLOP/s", "ms_per_call": round(cms, 1), "cores": threads,
                     "kind": "port", "sample": f"{ncall} call(s) of the same {T_}-token layer (all 256 experts), "
                                               "the reference's batched CPU expert path (weights decoded once per "
                                               "group of 4 pairs, cpu_dot_nl4_x4)", "host": cpu_host(threads)}
            if key == "prefill512":
                pre["prefill512_cpu_baseline"] = entry
            else:
                pre[key]["cpu_baseline"] = entry

    conv = None
    if not args.no_convert:
        log("converter: one layer of Q8_0 experts")
        conv = convert_bench(torch, qe_moe, 5, 0 if args.no_cpu_baseline else 4, threads)
        if conv.get("cpu_baseline"):
            conv["cpu_baseline"]["host"] = cpu_host(threads)
        torch.cuda.empty_cache()

    # ---------------- CPU baseline ----------------
    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline: {args.cpu_layers} distinct layers cycled over 40 steps, ~{args.cpu_seconds} s, {threads} threads")
        cpu_tok_s, cpu_sec, cpu_tok = cpu_baseline(args.cpu_layers, args.cpu_seconds, 100000, threads)
        cpu = {"value": round(cpu_tok_s, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
               "sample": f"{cpu_tok} tokens of B=1 decode through the 40-step stack ({args.cpu_layers} distinct seeded "
                         f"layers with all 256 experts each, cycled), full layer per step: norm, router, top-8, "
                         f"dispatch, int8 experts, Q8 shared, combine, residual; {cpu_sec:.2f} s of timed CPU work"}
        if threads != 12:  # the reference's default pool size (engine/qe.cpp:1201)
            t12, s12, n12 = cpu_baseline(args.cpu_layers, args.cpu_seconds / 2, 100000, 12)
            cpu["threads_12"] = {"value": round(t12, 3), "tokens": n12, "seconds": round(s12, 2)}
        cpu["host"] = cpu_host(threads)

    traffic = pmc_traffic(os.path.join(REPO, TRAFFIC_FILE))
    if dec is None:  # prefill-only run (profiling): no headline line
        print(json.dumps({**pre, "convert_layer_q8_0": conv, "cpu_baseline": cpu}), flush=True)
        return
    tok_s, ms, achieved, dec_avg_s, dec_bytes = dec["tok_s"], dec["ms"], dec["achieved"], dec["dec_avg_s"], dec["dec_bytes"]
    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic (seeded random-init weights of the config shapes)",
        "config": {"workload": "cfg2: 40-layer MoE-only stack, decode B=1, 1 token per step", "layers": N_LAYERS,
                   "tokens_per_step": 1, "experts": 256, "top_k": 8, "hip_graph": dec["graph_used"]},
        "hbm_gbs": round(N_LAYERS * LAYER_BYTES_B1 * tok_s / 1e9, 2),
        "hbm_frac": round(N_LAYERS * LAYER_BYTES_B1 * tok_s / HBM_PEAK, 4),
        **pre,
        "roofline": {"kernel": "k_decode (persistent: 40 layers x norm, router, top-8, experts, shared, combine)",
                     "bound": "hbm", "achieved": round(achieved / 1e9, 2), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4),
                     "traffic": None if traffic is None else round(traffic), "traffic_source": TRAFFIC_FILE,
                     "bytes_per_launch": dec_bytes,
                     "avg_us": round(dec_avg_s * 1e6, 3),
                     "avg_us_source": "timed region / steps (one k_decode launch per step, HIP events on its stream)"},
        "event_profiler_pass": dec["kernels"],
        "cfg0_decode_b1_layer": dec["cfg0"],
        "cfg1_decode_b8_zipf_layer": dec["cfg1"],
        "stack40_b8": dec["stack40_b8"],
        "layer_small_batch": {"note": "one layer per call, T tokens, no bias, calls rotated over 40 layers", **dec["small_t"]},
        "convert_layer_q8_0": conv,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
