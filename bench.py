"""Benchmark of the MI355X quantized-linear backend for janis.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu-baseline] [--quick]

Workload (the configuration the headline metric is quoted on): the decode
linears of a Qwen3-8B-shaped model at batch 1 -- 36 layers of
    qkv  4096 -> 4096+1024+1024   (q_proj, k_proj, v_proj as one launch; they share x)
    o    4096 -> 4096
    gate+up 4096 -> 2 x 12288     (one launch)
    down 12288 -> 4096
plus lm_head 4096 -> 151936, 4-bit affine group 64, bf16 scales/biases/x/y,
synthetic random weights resident in HBM (4.26 GB of packed weights). One
"step" is one token: the 145 launches in order, replayed from a HIP graph.

Printed: one JSON line with
    value     aggregate algorithmic HBM GB/s over the step
    tok_s     decode tok/s of the linears (1 / step time)
    roofline  for the dominant kernel, from HIP events on the launch stream
    cpu_baseline  janis's AVX2 per-channel kernel (restated in oracle/) on the
              host cores, on a bounded sample of the same workload
and per-shape, prefill (MFMA) and MoE-gather figures under "extra".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the dominant kernel, from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE over `bench.py --pmc-workload`, each scaled by what the counter reads
# for a 256 MiB copy in the same run (FETCH_SIZE x2.0, WRITE_SIZE x1.0). Re-measure
# after changing the kernel; the summary sits in profiles/.
DOMINANT_TRAFFIC_BYTES = 26917793
BF16_MFMA_PEAK_TFLOPS = 2500.0
HIDDEN, INTER, VOCAB, LAYERS, GS = 4096, 12288, 151936, 36, 64


def qbytes(n: int, k: int, bits: int = 4) -> int:
    """Algorithmic bytes of one g64 qmv: codes + bf16 scales/biases + x + y."""
    return n * k * bits // 8 + 4 * n * (k // GS) + 2 * k + 2 * n


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true", help="skip the extra per-config figures")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--decode-step", type=int, default=0, metavar="CTX",
                    help="profiling workload: only the config-4 decode step at context CTX (graph "
                         "replays, warmup + steps); prints one line to stderr")
    ap.add_argument("--fused-only", action="store_true",
                    help="with --decode-step: skip the reference's unfused call sequence (profiles of the fused "
                         "step alone)")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="eager launches for rocprofv3 --pmc: a 256 MiB copy (counter calibration), "
                         "then one pass of the dominant kernel's launches; prints nothing else")
    ap.add_argument("--shapes-workload", action="store_true",
                    help="eager launches for rocprofv3: each decode shape (qkv, o, gate_up, down, lm_head) "
                         "3 times on distinct weights, in that order")
    ap.add_argument("--prefill-workload", type=int, default=0, metavar="M",
                    help="eager launches for rocprofv3: the config-2 prefill products (gate_up 12288x4096, "
                         "down 4096x12288) at M rows, 3 times each")
    ap.add_argument("--dominant-workload", action="store_true",
                    help="profiling workload: only the roofline kernel's graph (36 layers x q/k/v, o, gate+up), "
                         "warmup + steps replays, the same graph bench.py times for `roofline`; prints one line "
                         "to stderr")
    ap.add_argument("--f32-workload", action="store_true",
                    help="eager launches for rocprofv3: one token of the config-1 linears with fp32 x (the "
                         "activation dtype of the reference's unchanged model code), then the same with bf16 x")
    ap.add_argument("--moe-workload", type=int, default=0, metavar="T",
                    help="eager launches for rocprofv3: the config-3 expert MLP (jh_moe_swiglu, Qwen3-30B-A3B "
                         "experts, top-8) at T tokens over 4 layers' expert stacks, 3 passes")
    ap.add_argument("--ceiling-workload", action="store_true",
                    help="profiling workload: the launch-ceiling measurements only (empty-kernel graph nodes, "
                         "re-reads after a 1 GiB read of other memory, the 2 GiB read and 1 GiB copy); prints "
                         "them to stderr")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this backend is measured on one GPU; --gpus N > 1 is not "
                                   "supported: this build measures one GPU (the path would shard "
                                   "by output rows, and MoE by expert)"}))
        return 2

    import torch

    from janis_amd.engine import BF16, F32, I32, U32, HipBackend

    dev = torch.device("cuda:0")
    torch.manual_seed(1234)
    hip = HipBackend(0)
    log("device:", hip.EngineInfo())

    def qweight(n, k, lead=(), bits=4):
        shape = (*lead, n, k * bits // 32)
        w = torch.randint(-2**31, 2**31 - 1, shape, dtype=torch.int32, device=dev)
        s = (torch.randn((*lead, n, k // GS), device=dev).abs() * 0.02).to(torch.bfloat16)
        b = (-float(1 << (bits - 1)) * s.float() + torch.randn((*lead, n, k // GS), device=dev) * 1e-3
             ).to(torch.bfloat16)
        return (hip.Wrap(w.data_ptr(), shape, U32, keep=w),
                hip.Wrap(s.data_ptr(), s.shape, BF16, keep=s),
                hip.Wrap(b.data_ptr(), b.shape, BF16, keep=b))

    def bf16(shape, randn=True):
        t = torch.randn(shape, device=dev).to(torch.bfloat16) if randn else \
            torch.empty(shape, device=dev, dtype=torch.bfloat16)
        return hip.Wrap(t.data_ptr(), shape, BF16, keep=t)

    # ---- weights and activations of the 36-layer sequence ---------------------------
    t0 = time.time()
    shapes = {"qkv": (HIDDEN + 2 * 1024, HIDDEN), "o": (HIDDEN, HIDDEN),
              "gate_up": (2 * INTER, HIDDEN), "down": (HIDDEN, INTER)}
    layers = [{name: qweight(n, k) for name, (n, k) in shapes.items()} for _ in range(LAYERS)]
    head = qweight(VOCAB, HIDDEN)
    x_h, x_attn, x_ffn = bf16((1, HIDDEN)), bf16((1, HIDDEN)), bf16((1, INTER))
    ys = {name: bf16((1, n), randn=False) for name, (n, k) in shapes.items()}
    y_head = bf16((1, VOCAB), randn=False)

    def f32(shape, randn=True):
        t = torch.randn(shape, device=dev) if randn else torch.empty(shape, device=dev)
        return hip.Wrap(t.data_ptr(), shape, F32, keep=t)

    # fp32 activations, the dtype janis's unchanged model code hands the products
    # (Dequantize returns F32 and every operator keeps its input's dtype)
    xin32 = {"qkv": f32((1, HIDDEN)), "o": f32((1, HIDDEN)), "gate_up": None, "down": f32((1, INTER))}
    xin32["gate_up"] = xin32["qkv"]
    ys32 = {name: f32((1, n), randn=False) for name, (n, k) in shapes.items()}
    y_head32 = f32((1, VOCAB), randn=False)
    torch.cuda.synchronize()
    log(f"weights ready in {time.time() - t0:.1f}s")
    xin = {"qkv": x_h, "o": x_attn, "gate_up": x_h, "down": x_ffn}

    def launch(name, wsb, x, y):
        w, s, b = wsb
        hip.QuantMatmul(x, w, s, b, True, GS, 4, out=y)

    def sequence():
        for L in layers:
            for name in ("qkv", "o", "gate_up", "down"):
                launch(name, L[name], xin[name], ys[name])
        launch("lm_head", head, x_h, y_head)

    def sequence_f32():
        for L in layers:
            for name in ("qkv", "o", "gate_up", "down"):
                launch(name, L[name], xin32[name], ys32[name])
        launch("lm_head", head, xin32["qkv"], y_head32)

    def token_stages():
        # the weight bytes (codes, bf16 scales and biases) of each launch of the token, in order
        return [int(0.5625 * n * k) for _ in range(LAYERS) for n, k in shapes.values()] + \
            [int(0.5625 * VOCAB * HIDDEN)]

    bytes_layer = sum(qbytes(n, k) for n, k in shapes.values())
    bytes_token = LAYERS * bytes_layer + qbytes(VOCAB, HIDDEN)
    n_launch = LAYERS * 4 + 1

    def capture(fn, keep=False):
        g = torch.cuda.CUDAGraph(keep_graph=keep)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            hip.SetStream(s.cuda_stream)
            fn()  # warm the launch path outside the graph
            torch.cuda.synchronize()
        with torch.cuda.graph(g):
            hip.SetStream(torch.cuda.current_stream().cuda_stream)
            fn()
        hip.SetStream(torch.cuda.current_stream().cuda_stream)
        if keep:
            g.instantiate()
        torch.cuda.synchronize()
        return g

    def time_graph(g, steps, warmup):
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(steps):
            g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps  # ms per replay

    if args.ceiling_workload:
        res = memory_floors(torch, dev, capture, time_graph, {}, token_stages())
        log("ceiling workload:", json.dumps(res))
        hip.Close()
        return 0

    if args.decode_step:
        res = decode_step_figures(hip, torch, dev, capture, time_graph, args, contexts=(args.decode_step,))
        log("decode step only:", res)
        hip.Close()
        return 0

    if args.shapes_workload:
        # calibration for FETCH_SIZE/WRITE_SIZE: a plain copy of 256 MiB first
        src = torch.empty(1 << 28, dtype=torch.uint8, device=dev).fill_(1)
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        hip.SetStream(torch.cuda.current_stream().cuda_stream)
        for name in ("qkv", "o", "gate_up", "down"):
            for L in layers[:3]:
                launch(name, L[name], xin[name], ys[name])
        for _ in range(3):
            launch("lm_head", head, x_h, y_head)
        torch.cuda.synchronize()
        log("shapes workload done")
        hip.Close()
        return 0

    if args.f32_workload:
        hip.SetStream(torch.cuda.current_stream().cuda_stream)
        sequence_f32()
        sequence()
        torch.cuda.synchronize()
        log("f32 workload done")
        hip.Close()
        return 0

    if args.moe_workload:
        from janis_amd import synth
        from janis_amd.engine import F32, I32
        E, H, I, K, T = 128, 2048, 768, 8, args.moe_workload
        stacks = [{"gate": qweight(I, H, (E,)), "up": qweight(I, H, (E,)), "down": qweight(H, I, (E,))}
                  for _ in range(4)]
        idx_np, sc_np = synth.route(77 + T, T, E, K)
        it, sct = torch.from_numpy(idx_np).to(dev), torch.from_numpy(sc_np).to(dev)
        idx = hip.Wrap(it.data_ptr(), tuple(idx_np.shape), I32, keep=it)
        scores = hip.Wrap(sct.data_ptr(), tuple(sc_np.shape), F32, keep=sct)
        xs = bf16((T, H))
        ot = torch.empty((T, H), device=dev, dtype=torch.float32)
        out = hip.Wrap(ot.data_ptr(), (T, H), F32, keep=ot)
        hip.SetStream(torch.cuda.current_stream().cuda_stream)
        for _ in range(3):
            for st in stacks:
                hip.MoeSwiGLU(xs, st["gate"], st["up"], st["down"], idx, scores, GS, 4, out=out)
        torch.cuda.synchronize()
        log(f"moe workload T={T} done")
        hip.Close()
        return 0

    if args.prefill_workload:
        hip.SetStream(torch.cuda.current_stream().cuda_stream)
        m = args.prefill_workload
        for n, k in ((12288, HIDDEN), (HIDDEN, INTER)):
            copies = [qweight(n, k) for _ in range(3)]
            x, y = bf16((m, k)), bf16((m, n), randn=False)
            for c in copies:
                hip.QuantMatmul(x, *c, True, GS, 4, out=y)
            torch.cuda.synchronize()
            del copies
        log(f"prefill workload M={m} done")
        hip.Close()
        return 0

    if args.pmc_workload:
        # calibration: a plain copy of known size (reads and writes 256 MiB)
        src = torch.empty(1 << 28, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        hip.SetStream(torch.cuda.current_stream().cuda_stream)
        for L in layers:
            for name in ("qkv", "o", "gate_up"):
                launch(name, L[name], xin[name], ys[name])
        torch.cuda.synchronize()
        log("pmc workload done")
        hip.Close()
        return 0

    if args.dominant_workload:
        def dominant_graph():
            for L in layers:
                for name in ("qkv", "o", "gate_up"):
                    launch(name, L[name], xin[name], ys[name])
        g = capture(dominant_graph)
        ms = time_graph(g, args.steps, args.warmup)
        log(f"dominant workload: {ms * 1e3 / (3 * LAYERS):.3f} us per launch")
        hip.Close()
        return 0

    # ---- headline: the whole token ------------------------------------------------------
    g_seq = capture(sequence)
    ms_step = time_graph(g_seq, args.steps, args.warmup)
    gbs = bytes_token / (ms_step * 1e-3) / 1e9
    tok_s = 1000.0 / ms_step
    log(f"sequence: {ms_step * 1e3:.1f} us/token, {gbs:.0f} GB/s, {tok_s:.0f} tok/s")
    # the same token with fp32 x and fp32 y (x rounded to bf16 in the tiles' registers)
    g_f32 = capture(sequence_f32)
    ms_f32 = time_graph(g_f32, args.steps, args.warmup)
    del g_f32
    bytes_f32 = bytes_token + LAYERS * sum(2 * (n + k) for n, k in shapes.values()) + 2 * (VOCAB + HIDDEN)
    f32_line = {"us_per_token": round(ms_f32 * 1e3, 1), "tok_s": round(1000.0 / ms_f32, 1),
                "GB_s": round(bytes_f32 / (ms_f32 * 1e-3) / 1e9, 1), "vs_bf16_x": round(ms_step / ms_f32, 4),
                "note": "config 1 with fp32 x and y (the dtype flow of the reference's unchanged model code); "
                        "algorithmic bytes count the 4-byte x and y"}
    log("sequence, fp32 x:", f32_line)

    # ---- per shape, rotating at least 64 distinct copies and 600 MB (the 256 MB ----------
    # memory-side cache cannot hold them): the 36 layers' copies plus fresh ones
    def n_rotate(n, k):
        return max(64, -(-600_000_000 // qbytes(n, k)))

    per_shape = {}
    for name, (n, k) in shapes.items():
        ws = [L[name] for L in layers] + [qweight(n, k) for _ in range(n_rotate(n, k) - LAYERS)]
        g = capture(lambda name=name, ws=ws: [launch(name, w, xin[name], ys[name]) for w in ws])
        ms = time_graph(g, max(5, args.steps // 2), 3) / len(ws)
        per_shape[name] = {"N": n, "K": k, "us": round(ms * 1e3, 2),
                           "GB_s": round(qbytes(n, k) / (ms * 1e-3) / 1e9, 1), "copies_rotated": len(ws)}
        del g, ws
    g = capture(lambda: launch("lm_head", head, x_h, y_head))
    ms = time_graph(g, max(5, args.steps // 2), 3)
    per_shape["lm_head"] = {"N": VOCAB, "K": HIDDEN, "us": round(ms * 1e3, 2),
                            "GB_s": round(qbytes(VOCAB, HIDDEN) / (ms * 1e-3) / 1e9, 1)}
    del g
    # q_proj and k_proj / v_proj as the reference's separate linears (config 1 times
    # each shape separately), rotated the same way
    for name, (n, k) in {"q_proj": (HIDDEN, HIDDEN), "k_proj": (1024, HIDDEN)}.items():
        copies = [qweight(n, k) for _ in range(n_rotate(n, k))]
        yq = bf16((1, n), randn=False)
        g = capture(lambda copies=copies, yq=yq: [hip.QuantMatmul(x_h, *c, True, GS, 4, out=yq) for c in copies])
        ms = time_graph(g, max(5, args.steps // 2), 3) / len(copies)
        per_shape[name] = {"N": n, "K": k, "us": round(ms * 1e3, 2),
                           "GB_s": round(qbytes(n, k) / (ms * 1e-3) / 1e9, 1), "copies_rotated": len(copies)}
        if name == "k_proj":
            per_shape[name]["note"] = "v_proj has the same shape"
        del g, copies
    # the plain-read floor of each shape's bytes (one launch reading them, nothing else)
    floors = memory_floors(torch, dev, capture, time_graph, {nm: qbytes(v["N"], v["K"]) for nm, v in per_shape.items()},
                           token_stages())
    for nm, v in per_shape.items():
        f = floors["floors"][nm]
        v["floor_us"] = f["us"]
        v["vs_floor"] = round(v["us"] / f["us"], 3)
    log("per shape:", per_shape)

    # ---- the same shapes with 8-bit codes (MLX's other affine width), rotated as above --
    per_shape_8 = {}
    for name, (n, k) in shapes.items():
        copies = [qweight(n, k, bits=8) for _ in range(max(64, -(-600_000_000 // qbytes(n, k, 8))))]
        g = capture(lambda name=name, copies=copies: [
            hip.QuantMatmul(xin[name], w, s_, b_, True, GS, 8, out=ys[name]) for (w, s_, b_) in copies])
        ms = time_graph(g, max(5, args.steps // 2), 3) / len(copies)
        per_shape_8[name] = {"N": n, "K": k, "us": round(ms * 1e3, 2),
                             "GB_s": round(qbytes(n, k, 8) / (ms * 1e-3) / 1e9, 1), "copies_rotated": len(copies)}
        del g, copies
    torch.cuda.synchronize()
    log("per shape, 8-bit:", per_shape_8)

    # ---- dominant kernel: the K=4096 GEMV tile (qkv, o, gate_up; ~69% of the step) -----
    # Events bracket a graph of exactly that kernel's launches, back to back, in the
    # sequence's order; achieved = their algorithmic bytes / their time per launch.
    dom_names = ("qkv", "o", "gate_up")

    def dominant_only():
        for L in layers:
            for name in dom_names:
                launch(name, L[name], xin[name], ys[name])

    g = capture(dominant_only)
    ms_dom = time_graph(g, args.steps, args.warmup)
    del g
    n_dom = LAYERS * len(dom_names)
    bytes_dom = LAYERS * sum(qbytes(*shapes[n]) for n in dom_names)
    dom_gbs = bytes_dom / (ms_dom * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": DOMINANT_TRAFFIC_BYTES,
                "traffic_source": "rocprofv3 --pmc FETCH_SIZE (x2.0) + WRITE_SIZE, "
                                  "profiles/qmv_bf16x_k4096_traffic.md",
                "kernel": "qmv_bf16x_kernel, K=4096 decode GEMV tiles <32,1,4,4> (qkv, gate_up) and <32,1,2,4> (o)",
                "launches_per_step": n_dom, "avg_launch_us": round(ms_dom * 1e3 / n_dom, 3),
                "algorithmic_bytes_per_launch": bytes_dom // n_dom}

    extra = {"config1_f32_x": f32_line, "per_shape": per_shape, "per_shape_8bit": per_shape_8,
             "launches_per_token": n_launch,
             "bytes_per_token": bytes_token, "hbm_measured": floors["hbm"],
             "read_floors": floors["floors"], "launch_ceiling": floors["ceiling"]}

    if not args.quick:
        extra.update(prefill_and_moe(hip, torch, dev, qweight, bf16, capture, time_graph, args))
        extra.update(decode_step_figures(hip, torch, dev, capture, time_graph, args))

    # ---- CPU baseline --------------------------------------------------------------------
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_seconds, bytes_token)

    out = {
        "metric": "4-bit qmv HBM GB/s (% of peak) + Qwen3-8B-shape decode tok/s, 1 MI355X",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 codes, bf16 act, fp32 acc",
        "data": "synthetic (random 4-bit codes, |N(0,1)|*0.02 bf16 scales, N(0,1) bf16 x)",
        "config": {"workload": "qwen3_8b_decode_linears_36L_plus_lm_head", "batch": 1,
                   "hidden": HIDDEN, "intermediate": INTER, "vocab": VOCAB, "layers": LAYERS,
                   "bits": 4, "group_size": GS, "launches": n_launch, "graph": True},
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "tok_s": round(tok_s, 1),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)
    hip.Close()
    return 0


def prefill_and_moe(hip, torch, dev, qweight, bf16, capture, time_graph, args):
    """Config 2 (prefill qmm, MFMA) and config 3 (MoE gather, whole expert MLP) figures."""
    from janis_amd import synth
    from janis_amd.engine import F32, I32

    res = {}
    # prefill: gate_up 4096->12288 and down 12288->4096 at M in {128, 512, 2048}
    pre = {}
    for name, (n, k) in {"gate_up": (12288, 4096), "down": (4096, 12288)}.items():
        # 24 copies (680 MB) rotated, more than the 256 MB memory-side cache holds
        copies = [qweight(n, k) for _ in range(24)]
        for m in (128, 512, 2048):
            x = bf16((m, k))
            y = bf16((m, n), randn=False)
            g = capture(lambda: [hip.QuantMatmul(x, *c, True, GS, 4, out=y) for c in copies])
            ms = time_graph(g, 5, 2) / len(copies)
            fl = 2.0 * m * n * k
            pre[f"{name}_M{m}"] = {"us": round(ms * 1e3, 1), "TFLOP_s": round(fl / (ms * 1e-3) / 1e12, 1),
                                   "mfma_frac": round(fl / (ms * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS, 4)}
            del g
        # a few rows (batched decode of several sequences, a short draft to
        # verify): on these matrices (2^24 weights and more) the multi-row decode
        # GEMV takes 2..4 rows (2 for down), HBM-bound on the weights, and the
        # MFMA tile's 32/64-row blocks the rest
        few = {}
        for m in ((2, 4, 8, 16, 32, 64) if k == 4096 else (2, 4, 16, 32, 64)):
            x = bf16((m, k))
            y = bf16((m, n), randn=False)
            g = capture(lambda: [hip.QuantMatmul(x, *c, True, GS, 4, out=y) for c in copies])
            ms = time_graph(g, 5, 2) / len(copies)
            byts = 0.5625 * n * k + 2 * m * (n + k)
            few[f"M{m}"] = {"us": round(ms * 1e3, 2), "GB_s": round(byts / (ms * 1e-3) / 1e9, 1)}
            del g
        pre[f"{name}_few_rows"] = few
        del copies
    res["prefill_qmm"] = pre
    log("prefill:", pre)

    # MoE: Qwen3-30B-A3B experts (E=128, hidden 2048, inter 768), top-8
    E, H, I, K = 128, 2048, 768, 8
    moe = {}
    # 32 layers of expert stacks (32 x 340 MB) rotated: even batch 1 (8 experts,
    # 21 MB per layer) then touches 680 MB, more than the 256 MB memory-side cache
    nl = 32
    stacks = [{"gate": qweight(I, H, (E,)), "up": qweight(I, H, (E,)), "down": qweight(H, I, (E,))}
              for _ in range(nl)]
    for T in (1, 16):
        idx_np, _ = synth.route(77 + T, T, E, K)
        U = len(set(idx_np.reshape(-1).tolist()))
        it = torch.from_numpy(idx_np).to(dev)
        idx = hip.Wrap(it.data_ptr(), tuple(idx_np.shape), I32, keep=it)
        xg = bf16((T, 1, 1, H))
        hg = bf16((T, K, 1, I))
        yg, yu = bf16((T, K, 1, I), randn=False), bf16((T, K, 1, I), randn=False)
        yd = bf16((T, K, 1, H), randn=False)

        def moe_layers():
            for st in stacks:
                hip.GatherQuantMatmul(xg, *st["gate"], idx, True, GS, 4, out=yg)
                hip.GatherQuantMatmul(xg, *st["up"], idx, True, GS, 4, out=yu)
                hip.GatherQuantMatmul(hg, *st["down"], idx, True, GS, 4, out=yd)

        g = capture(moe_layers)
        ms = time_graph(g, 10, 3) / nl
        per_expert = 3 * (I * H // 2 + 4 * I * (H // GS))  # packed codes + scales/biases of one expert
        byt = U * per_expert + 2 * T * H + 2 * T * K * (2 * I + H) + 2 * T * K * I
        bucketing = T * K > 32  # past 32 pairs each call buckets in a launch of its own
        moe[f"T{T}"] = {"unique_experts": U, "us_per_layer": round(ms * 1e3, 2),
                        "GB_s": round(byt / (ms * 1e-3) / 1e9, 1), "launches_per_layer": 6 if bucketing else 3}
        del g

        # the whole expert MLP (gate+up SwiGLU, down with the score-weighted sum)
        _, sc_np = synth.route(77 + T, T, E, K)
        sct = torch.from_numpy(sc_np).to(dev)
        scores = hip.Wrap(sct.data_ptr(), tuple(sc_np.shape), F32, keep=sct)
        xs = bf16((T, H))
        ot = torch.empty((T, H), device=dev, dtype=torch.float32)
        out = hip.Wrap(ot.data_ptr(), (T, H), F32, keep=ot)

        def moe_fused():
            for st in stacks:
                hip.MoeSwiGLU(xs, st["gate"], st["up"], st["down"], idx, scores, GS, 4, out=out)

        g = capture(moe_fused)
        ms = time_graph(g, 10, 3) / nl
        byt = U * per_expert + 2 * T * H + 2 * 2 * T * K * I + 4 * T * H
        moe[f"T{T}_swiglu"] = {"unique_experts": U, "us_per_layer": round(ms * 1e3, 2),
                               "GB_s": round(byt / (ms * 1e-3) / 1e9, 1), "launches_per_layer": 3 if bucketing else 2,
                               "note": "jh_moe_swiglu: [bucketing] + gate/up SwiGLU (clearing out) + down combine"}
        del g
    res["moe_gather"] = moe
    log("moe:", moe)
    del stacks
    torch.cuda.empty_cache()
    return res


def graph_kernel_nodes(graph) -> int:
    """Kernel nodes of a captured HIP graph (hipGraphGetNodes / hipGraphNodeGetType)."""
    import ctypes

    rt = ctypes.CDLL("libamdhip64.so")
    n = ctypes.c_size_t(0)
    if rt.hipGraphGetNodes(ctypes.c_void_p(graph), None, ctypes.byref(n)) != 0:
        return -1
    nodes = (ctypes.c_void_p * n.value)()
    if rt.hipGraphGetNodes(ctypes.c_void_p(graph), nodes, ctypes.byref(n)) != 0:
        return -1
    kinds = [ctypes.c_int(0) for _ in range(n.value)]
    for i in range(n.value):
        if rt.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(kinds[i])) != 0:
            return -1
    return sum(1 for k in kinds if k.value == 0)  # hipGraphNodeTypeKernel


def decode_step_figures(hip, torch, dev, capture, time_graph, args, contexts=(512, 8192)):
    """Config 4: the whole Qwen3-8B-architecture decode step (36 layers: RMSNorm,
    q/k/v product, per-head q/k RMSNorm, RoPE, KV append, SDPA over the cache, o
    product, residual, RMSNorm, gate/up product, SiLU*mul, down product,
    residual; final norm, lm_head, argmax) on random-init 4-bit weights, bf16 KV
    caches filled with N(0,1) to ctx tokens, one new token at position ctx, as
    one graph of the engine-level operators (janis_amd/qwen3_decode.py, fused:
    norms in the products they feed, residual adds in the products' epilogues)."""
    from janis_amd.engine import I32
    from janis_amd.qwen3_decode import Qwen3Config, decode_step, random_model

    cfg = Qwen3Config()
    t0 = time.time()
    m, _ = random_model(hip, cfg, max(contexts) + 1, seed=4, torch=torch, dev=dev)
    for L in m.layers:
        L.k_cache._keep.normal_()
        L.v_cache._keep.normal_()
    torch.cuda.synchronize()
    log(f"decode-step model ready in {time.time() - t0:.1f}s")
    tok = torch.tensor([1234], dtype=torch.int32, device=dev)
    tt = hip.Wrap(tok.data_ptr(), (1,), I32, keep=tok)
    arena = hip.make_arena(64 << 20)
    H, Hq, Hk, Dh, I = cfg.hidden, cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.inter
    per_layer = (qbytes((Hq + 2 * Hk) * Dh, H) + qbytes(H, Hq * Dh) + qbytes(2 * I, H) + qbytes(H, I))
    weights = cfg.layers * per_layer + qbytes(cfg.vocab, H) + (H // 2 + 4 * (H // GS))  # + one embedding row
    res = {}
    for ctx in contexts:
        def fn(ctx=ctx):
            with hip.use_arena(arena):
                decode_step(hip, m, tt, ctx)
        g = capture(fn, keep=True)
        launches = graph_kernel_nodes(g.raw_cuda_graph())
        ms = time_graph(g, max(5, args.steps // 4), 3)
        kv = cfg.layers * 2 * Hk * (ctx + 1) * Dh * 2
        res[f"ctx{ctx}"] = {"us_per_token": round(ms * 1e3, 1), "tok_s": round(1000.0 / ms, 1),
                            "GB_s": round((weights + kv) / (ms * 1e-3) / 1e9, 1), "kv_bytes": kv,
                            "launches_per_token": launches}
        del g
    if getattr(args, "fused_only", False):
        log("decode step:", res)
        del m, arena
        torch.cuda.empty_cache()
        return {"qwen3_8b_decode_step": res}
    # The reference's own call sequence (qwen/block.go, qwen/attention.go,
    # qwen/mlp.go, qwen/cache.go: one engine call per operator, F32 activations,
    # KVCache.Update's cast to F16 caches) at the smallest context, in a graph:
    # what unchanged janis model code gets through the plain binding.
    import copy

    from janis_amd.engine import F16
    ctx = min(contexts)
    m16 = copy.copy(m)
    m16.layers = []
    for L in m.layers:
        L2 = copy.copy(L)
        for name in ("k_cache", "v_cache"):
            t = getattr(L, name)._keep[:, :, :ctx + 8].to(torch.float16).contiguous()
            setattr(L2, name, hip.Wrap(t.data_ptr(), tuple(t.shape), F16, keep=t))
        m16.layers.append(L2)
    torch.cuda.synchronize()

    def ref_calls():
        with hip.use_arena(arena):
            decode_step(hip, m16, tt, ctx, fused=False)
    g = capture(ref_calls, keep=True)
    launches = graph_kernel_nodes(g.raw_cuda_graph())
    ms = time_graph(g, max(5, args.steps // 4), 3)
    kv = cfg.layers * 2 * Hk * (ctx + 1) * Dh * 2
    res[f"ctx{ctx}_reference_calls_f32_f16cache"] = {
        "us_per_token": round(ms * 1e3, 1), "tok_s": round(1000.0 / ms, 1),
        "GB_s": round((weights + kv) / (ms * 1e-3) / 1e9, 1), "launches_per_token": launches,
        "note": "decode_step(fused=False): the reference's operator calls one by one with its dtype flow"}
    del g, m16
    log("decode step:", res)
    del m, arena
    torch.cuda.empty_cache()
    return {"qwen3_8b_decode_step": res}


def memory_floors(torch, dev, capture, time_graph, sizes, stages):
    """Measured HBM figures from bench.py's own kernels (janis_amd/libjanis_bench.so):
    a 1 GiB device copy and a 2 GiB read (the device's bandwidth beside the 8 TB/s
    specification), and for each byte count in `sizes` the fastest single launch that
    only reads that many bytes -- a graph of launches over distinct windows of a 2 GiB
    buffer (at least 64 windows and 600 MB where the buffer holds them, so the 256 MB
    memory-side cache cannot serve them), best of 1/2/4
    blocks per CU and 4/8/16 loads per lane in flight. That is the floor a decode
    product of those bytes can reach in one launch. `stages`: the byte counts of a
    token's launches in order, for the chained-read figure of ceiling_figures."""
    import ctypes

    from janis_amd import build as jb

    L = ctypes.CDLL(jb.BENCH_LIB)
    L.jhb_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                           ctypes.c_void_p]
    L.jhb_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    L.jhb_read_cached.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    L.jhb_empty.argtypes = [ctypes.c_int, ctypes.c_void_p]
    L.jhb_barriers.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint,
                               ctypes.c_void_p, ctypes.c_void_p]
    L.jhb_read.restype = L.jhb_copy.restype = L.jhb_read_cached.restype = L.jhb_empty.restype = ctypes.c_int
    L.jhb_barriers.restype = ctypes.c_int
    L.jhb_chain_read.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_uint, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    L.jhb_chain_read.restype = ctypes.c_int
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    pool_bytes = 2 << 30
    pool = torch.empty(pool_bytes, dtype=torch.uint8, device=dev).fill_(7)
    sink = torch.zeros(64, dtype=torch.int32, device=dev)

    def reads(nb, blocks, unroll, n):
        st = torch.cuda.current_stream().cuda_stream
        for i in range(n):
            rc = L.jhb_read(pool.data_ptr() + i * nb, nb, sink.data_ptr(), blocks, unroll, st)
            if rc != 0:
                raise RuntimeError(f"jhb_read: {rc}")

    floors = {}
    for name, nbytes in sizes.items():
        nb = (int(nbytes) + 255) // 256 * 256
        n = max(1, min(pool_bytes // nb, max(64, -(-600_000_000 // nb))))
        best = None
        for bpc in (1, 2, 4):
            for unroll in (4, 8, 16):
                g = capture(lambda: reads(nb, bpc * cus, unroll, n))
                ms = time_graph(g, 10, 3) / n
                del g
                if best is None or ms < best[0]:
                    best = (ms, bpc, unroll)
        floors[name] = {"bytes": nb, "us": round(best[0] * 1e3, 2), "GB_s": round(nb / (best[0] * 1e-3) / 1e9, 1),
                        "blocks_per_cu": best[1], "loads_in_flight_per_lane": best[2], "launches_timed": n}
    ceiling = ceiling_figures(torch, L, pool, sink, capture, time_graph, cus, stages)
    # whole-buffer read and copy
    g = capture(lambda: reads(pool_bytes, 4 * cus, 8, 1))
    ms_read = time_graph(g, 10, 3)
    del g
    half = pool_bytes // 2

    def copy():
        rc = L.jhb_copy(pool.data_ptr() + half, pool.data_ptr(), half, 4 * cus, torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"jhb_copy: {rc}")

    g = capture(copy)
    ms_copy = time_graph(g, 10, 3)
    del g, pool
    torch.cuda.empty_cache()
    hbm = {"copy_GB_s": round(2 * half / (ms_copy * 1e-3) / 1e9, 1),
           "read_GB_s": round(pool_bytes / (ms_read * 1e-3) / 1e9, 1),
           "note": "1 GiB device copy (read + write bytes / time) and a 2 GiB read, one launch each, "
                   "janis_amd/csrc/bench_kernels.hip; the roofline's peak stays the 8 TB/s specification"}
    log("hbm measured:", hbm, "read floors:", floors)
    return {"hbm": hbm, "floors": floors, "ceiling": ceiling}


def ceiling_figures(torch, L, pool, sink, capture, time_graph, cus, stages):
    """What bounds one launch per linear, measured with bench.py's own kernels:
    - graph_node_us: a graph of 64 dependent launches of an empty kernel (1 and
      256 blocks), time per launch -- the fixed cost each extra kernel adds;
    - grid_barrier_us: a grid-wide barrier inside one launch (one block per CU,
      a counter in memory; relaxed, and with release/acquire ordering, which is
      what a persistent kernel needs between dependent stages on different
      XCDs), time per barrier;
    - reread: a buffer of S bytes read three times in a row right after a 1 GiB
      read of other memory (which leaves none of it in the 256 MB memory-side
      cache): the first two reads with one cache policy (non-temporal, as the
      decode products load weights, or the default), the third non-temporal.
      Events around each launch, median of 5 rounds. A second or third read
      faster than the first means that cache served it;
    - chained_read: a token's weight bytes (`stages`, each launch's bytes in
      order, laid out one after another in a buffer of their total) read as a
      graph of one read launch per stage (4 blocks per CU, 8 loads per lane in
      flight), against one persistent launch that reads every stage (an even
      share per block) with a grid-wide barrier between stages -- per-block
      arrival flags, one per 128-byte line -- and the next stage's first loads
      issued before each wait (one 512- or 1024-thread block per CU, 8 loads
      per lane), and against that launch with the whole token as one stage (its
      streaming rate without barriers); median of 5."""
    st = torch.cuda.current_stream().cuda_stream

    def chk(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {rc}")

    nodes = {}
    for blocks in (1, 256):
        g = capture(lambda blocks=blocks: [chk(L.jhb_empty(blocks, torch.cuda.current_stream().cuda_stream), "jhb_empty")
                                           for _ in range(64)])
        nodes[f"blocks_{blocks}"] = round(time_graph(g, 20, 5) * 1e3 / 64, 3)
        del g
    base = pool.data_ptr()
    flush_off = 1 << 30

    def read(off, nb, nt):
        if nt:
            chk(L.jhb_read(base + off, nb, sink.data_ptr(), 4 * cus, 8, st), "jhb_read")
        else:
            chk(L.jhb_read_cached(base + off, nb, sink.data_ptr(), 4 * cus, st), "jhb_read_cached")

    reread = {}
    for mb in (48, 160):
        nb = mb << 20
        for nt in (True, False):
            t1, t2, t3 = [], [], []
            for _ in range(5):
                read(flush_off, 1 << 30, True)
                read(flush_off, 1 << 30, False)
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
                ev[0].record()
                read(0, nb, nt)
                ev[1].record()
                read(0, nb, nt)
                ev[2].record()
                read(0, nb, True)
                ev[3].record()
                torch.cuda.synchronize()
                t1.append(ev[0].elapsed_time(ev[1]) * 1e3)
                t2.append(ev[1].elapsed_time(ev[2]) * 1e3)
                t3.append(ev[2].elapsed_time(ev[3]) * 1e3)
            med = [sorted(t)[2] for t in (t1, t2, t3)]
            reread[f"{mb}MB_{'nt' if nt else 'default'}"] = {
                "first_us": round(med[0], 2), "second_us": round(med[1], 2), "third_nt_us": round(med[2], 2),
                "first_TB_s": round(nb / med[0] / 1e6, 2), "third_TB_s": round(nb / med[2] / 1e6, 2)}
    # grid-wide barriers inside one launch (one 64-thread block per CU): the
    # per-stage synchronisation a persistent kernel would pay instead of a graph
    # node; time per barrier = (64-round launch - 1-round launch) / 63, median of 5
    cnt = torch.zeros(16, dtype=torch.int32, device=pool.device)
    barrier = {}
    for ordered in (0, 1):
        per = []
        failed = False
        for _ in range(5):
            ts = []
            for rounds in (1, 64):
                cnt.zero_()
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
                ev[0].record()
                chk(L.jhb_barriers(cnt.data_ptr(), cus, rounds, ordered, 1 << 22, cnt.data_ptr() + 32, st),
                    "jhb_barriers")
                ev[1].record()
                torch.cuda.synchronize()
                failed |= int(cnt[8].item()) != 0
                ts.append(ev[0].elapsed_time(ev[1]) * 1e3)
            per.append((ts[1] - ts[0]) / 63)
        barrier["acq_rel" if ordered else "relaxed"] = None if failed else round(sorted(per)[2], 3)
    chained = chained_read(torch, L, sink, capture, time_graph, cus, stages, chk) if stages else None
    out = {"graph_node_us": nodes, "grid_barrier_us": barrier, "reread": reread, "chained_read": chained,
           "note": "empty-kernel graph nodes; grid-wide barriers inside one launch (one block per CU); "
                   "re-reads after a 1 GiB read of other memory; a token's reads as one launch per stage "
                   "and as one persistent launch (janis_amd/csrc/bench_kernels.hip)"}
    log("ceiling:", out)
    return out


def chained_read(torch, L, sink, capture, time_graph, cus, stages, chk):
    """The `chained_read` figure of ceiling_figures."""
    import numpy as np

    sizes = [(int(b) + 255) // 256 * 256 for b in stages]
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    total = int(sum(sizes))
    buf = torch.empty(total, dtype=torch.uint8, device=sink.device)
    base = buf.data_ptr()
    tab = torch.tensor([[base + int(o), n // 16] for o, n in zip(offs, sizes)], dtype=torch.int64, device=sink.device)

    def graph_of_reads():
        st = torch.cuda.current_stream().cuda_stream
        for o, n in zip(offs, sizes):
            chk(L.jhb_read(base + int(o), n, sink.data_ptr(), 4 * cus, 8, st), "jhb_read")

    g = capture(graph_of_reads)
    per_stage_us = sorted(time_graph(g, 5, 2) * 1e3 for _ in range(5))[2]
    del g
    one = torch.tensor([[base, total // 16]], dtype=torch.int64, device=sink.device)
    flags = torch.zeros(32 * cus + 64, dtype=torch.int32, device=sink.device)
    fail_off = 32 * cus

    def chain_us(t, n, threads):
        ts, failed = [], False
        for _ in range(6):
            flags.zero_()
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record()
            chk(L.jhb_chain_read(t.data_ptr(), n, flags.data_ptr(), 1 << 20, flags.data_ptr() + 4 * fail_off,
                                 sink.data_ptr(), cus, threads, torch.cuda.current_stream().cuda_stream),
                "jhb_chain_read")
            ev[1].record()
            torch.cuda.synchronize()
            failed |= int(flags[fail_off].item()) != 0
            ts.append(ev[0].elapsed_time(ev[1]) * 1e3)
        return None if failed else round(sorted(ts[1:])[2], 1)

    chain = {}
    for threads in (512, 1024):
        chain[f"threads_{threads}"] = {"stages_us": chain_us(tab, len(sizes), threads),
                                       "one_stage_us": chain_us(one, 1, threads)}
    del buf, tab, one, flags
    torch.cuda.empty_cache()
    return {"stages": len(sizes), "bytes": total, "launch_per_stage_us": round(per_stage_us, 1),
            "launch_per_stage_TB_s": round(total / per_stage_us / 1e6, 3), "persistent_launch_us": chain}


def host_info() -> dict:
    """nproc, the cores this process may use, the CPU model and the L3 size."""
    info = {"nproc": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    info["cpu_model"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    # total L3: the size of each distinct L3 instance (by the CPUs sharing it)
    seen, total = set(), 0
    base = "/sys/devices/system/cpu"
    try:
        for cpu in sorted(os.listdir(base)):
            d = os.path.join(base, cpu, "cache", "index3")
            if not cpu.startswith("cpu") or not os.path.isdir(d):
                continue
            with open(os.path.join(d, "shared_cpu_list")) as f:
                key = f.read().strip()
            if key in seen:
                continue
            seen.add(key)
            with open(os.path.join(d, "size")) as f:
                sz = f.read().strip()
            mult = {"K": 1 << 10, "M": 1 << 20}.get(sz[-1:], 1)
            total += int(sz.rstrip("KM")) * mult
    except (OSError, ValueError):
        pass
    if total:
        info["l3_bytes"] = total
        info["l3_instances"] = len(seen)
    return info


def cpu_baseline(seconds: float, bytes_token: int):
    """janis's amd64 decode path -- the AVX2 per-channel kernel over parallelFor
    chunks (cpu/qmv_amd64.s, cpu/cpu.go:37-79), restated in oracle/ -- timed on
    the host cores of the GPU box over the same decode shapes: whole layers
    (qkv, o, gate_up, down) plus slices of lm_head, distinct random matrices
    totalling at least 4x the host's L3 (so every pass streams from DRAM, as
    the reference does on a real model), each read once per pass."""
    import numpy as np

    from oracle import oracle

    info = host_info()
    # 16 cores: the GPU box's CPU share for one GPU (its scheduler allots 16 per
    # GPU whatever nproc shows), so the parallelFor split runs over 16 workers
    cores = min(info["affinity"], 16)
    target = max(4 * info.get("l3_bytes", 256 << 20), 1 << 30)
    layer = [(6144, HIDDEN), (HIDDEN, HIDDEN), (2 * INTER, HIDDEN), (HIDDEN, INTER)]
    rng = np.random.default_rng(77)
    mats, byt = [], 0
    while byt < target:
        for n, k in layer + [(VOCAB // 8, HIDDEN)]:
            w = rng.integers(0, 1 << 32, size=(n, k // 8), dtype=np.uint32)
            sc = (np.abs(rng.standard_normal((n, k // GS))) * 0.02).astype(np.float32)
            bi = (-8.0 * sc + rng.standard_normal((n, k // GS)) * 1e-3).astype(np.float32)
            mats.append((w, sc, bi, k))
            byt += qbytes(n, k)
    xs = {k: rng.standard_normal(k).astype(np.float32) for k in (HIDDEN, INTER)}
    for w, sc, bi, k in mats[:5]:  # untimed warm-up (page faults, thread start)
        oracle.qmv_avx2_parallel(xs[k], w, sc, bi, GS, cores)
    t0 = time.perf_counter()
    passes = 0
    used = cores
    while True:
        for w, sc, bi, k in mats:
            _, used = oracle.qmv_avx2_parallel(xs[k], w, sc, bi, GS, cores)
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    gbs = byt * passes / el / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": int(used), "kind": "port",
            "avx2": bool(oracle.have_avx2_fma()),
            "tok_s_equiv": round(gbs * 1e9 / bytes_token, 2),
            "host": info,
            "sample": f"{passes} passes over {len(mats)} distinct matrices (whole Qwen3-8B decode layers + "
                      f"lm_head slices, {byt / 1e6:.0f} MB >= 4x L3), fp32 x, {el:.1f}s; "
                      f"{int(used)} workers = the box's 16-core share for one GPU"}


if __name__ == "__main__":
    sys.exit(main())
