#!/usr/bin/env python3
"""Benchmark of the entropy-gated precision path on one MI355X.

Metric: INT8/FP8 GEMM TOPS and softmax+entropy GB/s, as a
fraction of roofline, at 1024x4096x4096 on 1 GPU -- configs[0]'s shapes:
  * INT8 tier GEMM M=1024, K=4096, N=4096: activations fp16 N(0,1) quantised
    per row (the reference's dispatcher quantiser), weights fp16 N(0,0.02)
    quantised per output channel; int32 accumulate; fp16 dequant output.
  * FP8 e4m3 tier GEMM on the same inputs.
  * fused softmax + entropy over fp16 [1024, 4096], rows N(0, s),
    s uniform over {0.25, 1, 4, 16}.
A "step" is one launch of the INT8 GEMM on pre-quantised activations (the
reference's headline CubinEngine measurement); `value` is its TOPS.  The FP8
GEMM, the entropy kernel, the quantisers and the end-to-end launchers are
timed the same way and reported under "kernels".

Timing: W untimed warmup steps, then EXACTLY K steps between events recorded
on the stream the kernels run on, bracketed by torch.cuda.synchronize(); the
median of 5 such timed regions is reported (`value`, `ms_per_step`).  The
roofline figures divide the algorithmic work by the kernel's average launch
duration over the timed region of one replayed HIP graph holding the K
launches (the host-side gaps of an eager loop are left out; this is the
figure rocprofv3's per-dispatch durations agree with).  Each kernel is timed
twice: from K eager launches (the reference's own loop) and from one HIP graph
holding the K launches.  The GEMMs report the eager figure
(their launches keep the queue full; graph replay adds per-node overhead); the
6-9 us entropy and quantiser kernels report the graph figure (eager Python
launches of them are host-bound).  Both figures are in kernels.timings_us.
GEMM operands stay resident (as in the reference's loop); the HBM-bound
entropy kernel rotates through enough input/output buffers to exceed the
256 MB Infinity Cache ("cold", the roofline figure) and also reports the
same-buffer ("hot") rate.
cpu_baseline: the reference path's arithmetic as PyTorch CPU ops
(oracle/torch_cpu.py: INT8 with torch._int_mm, FP8 through f32, f32 entropy)
and the repository's C oracle, timed on this host's cores over a bounded
sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "triton-kernels-optimization_amd"))

METRIC = "INT8/FP8 GEMM TOPS & entropy GB/s (% roofline), 1024x4096x4096, 1 GPU"
PEAK_I8_TOPS = 5000.0          # MI355X dense int8 (5.0 POP/s)
PEAK_F8_TFLOPS = 5000.0        # MI355X dense fp8 (5.0 PFLOP/s)
PEAK_F16_TFLOPS = 2500.0       # MI355X dense fp16
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
M, K, N = 1024, 4096, 4096
ER, ES = 1024, 4096            # entropy rows x columns
COPY_BYTES = 256 << 20         # calibration copy for the FETCH_SIZE / WRITE_SIZE counters


def mixture_logits(rng, M: int, S: int, fractions=(0.2, 0.4, 0.4),
                   bands=((0.05, 0.36), (0.46, 1.62), (1.75, 7.5))):
    """Config 3's routing logits: fp16 [M, S] rows whose entropies fall ~20% below
    0.41, ~40% in [0.41, 1.68) and ~40% above 1.68 nats.  Each row is N(0,1)
    background plus one spike column; with spike mass p and background entropy
    H_b the row entropy is H(p) = -p ln p - (1-p) ln(1-p) + (1-p) H_b, which is
    solved for p by bisection toward a target drawn from the row's band.
    Returns (logits fp16, class per row)."""
    import numpy as np
    x = rng.standard_normal((M, S))
    m = x.max(axis=1, keepdims=True)
    e = np.exp(x - m)
    zb = e.sum(axis=1)
    pb = e / zb[:, None]
    hb = -(pb * np.log(pb)).sum(axis=1)
    cls = rng.choice(3, M, p=fractions)
    lo = np.array([b[0] for b in bands])[cls]
    hi = np.array([b[1] for b in bands])[cls]
    target = lo + (hi - lo) * rng.random(M)
    a, b = np.full(M, 1e-9), np.full(M, 1 - 1e-12)
    for _ in range(60):
        p = 0.5 * (a + b)
        h = -p * np.log(p) - (1 - p) * np.log1p(-p) + (1 - p) * hb
        a, b = np.where(h > target, p, a), np.where(h > target, b, p)
    p = 0.5 * (a + b)
    x[np.arange(M), rng.integers(0, S, M)] = m[:, 0] + np.log(p * zb / (1 - p))
    return x.astype(np.float16), cls


def parse():
    ap = argparse.ArgumentParser(description="entropy-gated path benchmark (1 GPU)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches only")
    ap.add_argument("--only", default="", help="comma list of kernels to time (profiling runs)")
    return ap.parse_args()


def time_steps(fn, steps: int, warmup: int, use_graph: bool, stream, repeats: int = 5, warm_s: float = 0.1):
    """ms per step of `fn` (which launches on `stream`): the median over
    `repeats` timed regions, each of exactly `steps` launches between events
    on `stream`, bracketed by torch.cuda.synchronize().  Untimed warmup: the
    `warmup` launches, then more until `fn` has kept the GPU busy for `warm_s`
    seconds: after the host-side setup between legs the GPU has idled, and it
    takes ~0.1 s of load to reach its steady clock (the C0 INT8 GEMM measured
    24.8, 23.0, then 22.2 us in three back-to-back timings straight after idle).
    A captured graph is likewise replayed for `warm_s` before the timed
    replays: the first replays of the run's first graph ran the C0 INT8 GEMM
    at ~25.5 us per launch against 22 us eager, the same after the warm-up."""
    import torch
    t0 = time.perf_counter()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < warm_s:
        for _ in range(max(1, warmup)):
            fn()
        torch.cuda.synchronize()
    graph = None
    if use_graph:
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for _ in range(steps):
                    fn()
            t1 = time.perf_counter()            # untimed replays, for warm_s as well
            while True:
                graph.replay()
                torch.cuda.synchronize()
                if time.perf_counter() - t1 >= warm_s:
                    break
        except Exception as e:                  # capture unsupported -> eager only
            print(f"# graph capture failed ({type(e).__name__}: {e}); timing eager launches", file=sys.stderr)
            graph = None
            torch.cuda.synchronize()
    times = []
    with torch.cuda.stream(stream):
        for _ in range(repeats):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record(stream)
            if graph is not None:
                graph.replay()
            else:
                for _ in range(steps):
                    fn()
            end.record(stream)
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end) / steps)
    times.sort()
    return times[len(times) // 2], graph is not None


def time_launches(fn, steps: int, warmup: int, stream) -> float:
    """Average duration (ms) of one launch of `fn`: every launch bracketed by
    its own pair of events on `stream`, so the gaps between launches are left
    out -- the per-launch figure the roofline divides into, comparable with
    the profiler's per-dispatch durations."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    with torch.cuda.stream(stream):
        for a, b in ev:
            a.record(stream)
            fn()
            b.record(stream)
        torch.cuda.synchronize()
    d = sorted(a.elapsed_time(b) for a, b in ev)
    return d[len(d) // 2]


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import entropy_engine as ee
    from entropy_engine import _lib as eel

    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.Stream(dev)
    only = set(filter(None, args.only.split(",")))
    rng = np.random.default_rng(0)

    # ---------------- inputs (generated on the CPU, copied once)
    A = torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32)).half()
    W = (torch.from_numpy(rng.standard_normal((N, K), dtype=np.float32)) * 0.02).half()
    sc = torch.from_numpy(rng.choice(np.float32([0.25, 1.0, 4.0, 16.0]), ER))
    L = (torch.from_numpy(rng.standard_normal((ER, ES), dtype=np.float32)) * sc[:, None]).half()
    with torch.cuda.stream(stream):
        a = A.to(dev)
        B_kn, b_scale = ee.quantize_weights_int8(W.to(dev))
        pw = ee.prepare_weight(B_kn, b_scale).materialize()
        a_i8, s_i8 = ee.quantize_activations(a, "dispatcher")
        a_f8, s_f8 = ee.quantize_activations(a, "fp8")
        c = torch.empty((M, N), dtype=torch.float16, device=dev)
        n_rot = 40                                                     # 40 x 16 MB > 2 x 256 MB MALL
        logits = [L.to(dev)] + [torch.empty_like(L, device=dev) for _ in range(n_rot - 1)]
        for t in logits[1:]:
            t.copy_(logits[0])
        probs = [torch.empty((ER, ES), dtype=torch.float16, device=dev) for _ in range(n_rot)]
        w16 = pw.f16
    torch.cuda.synchronize()

    ops = 2.0 * M * N * K
    ent_bytes = ER * ES * 2 * 2 + ER * 4                               # read fp16, write fp16 probs, write f32 H
    use_graph = not args.no_graph
    results = {}

    def run(name, fn, steps=args.steps, warmup=args.warmup, primary="graph", graph=True):
        """Times `fn` from eager launches and, unless --no-graph (or graph=False),
        from a replayed HIP graph of the K launches; "ms" is the `primary` one."""
        if only and name not in only:
            return None
        with torch.cuda.stream(stream):
            ms_eager, _ = time_steps(fn, steps, warmup, False, stream)
            ms_graph, g = time_steps(fn, steps, warmup, True, stream) if (use_graph and graph) else (None, False)
        use = "graph" if (primary == "graph" and g) else "eager"
        results[name] = {"ms": ms_graph if use == "graph" else ms_eager, "timing": use,
                         "ms_eager": ms_eager, "ms_graph": ms_graph}
        return results[name]["ms"]

    with torch.cuda.stream(stream):
        # headline: INT8 GEMM kernel on pre-quantised activations
        # GEMMs (26-50 us each) keep the queue full from eager launches, as in the
        # reference's own timing loop; graph replay adds per-node overhead on top.
        run("gemm_i8", lambda: ee.gemm("int8", a_i8, pw.i8, s_i8, pw.scale, out=c), primary="eager")
        i8_kernel = eel.lib().ee_last_kernel().decode()
        run("gemm_f8", lambda: ee.gemm("fp8", a_f8, pw.f8, s_f8, pw.scale, out=c), primary="eager")
        run("gemm_f16w8", lambda: ee.gemm("fp16", a, w16, out=c), primary="eager")
        rot = {"i": 0}

        def ent_cold():
            i = rot["i"] % n_rot
            rot["i"] += 1
            ee.softmax_entropy(logits[i], out_probs=probs[i])

        run("softmax_entropy_cold", ent_cold, steps=n_rot * max(1, args.steps // n_rot), warmup=n_rot)
        ent_kernel = eel.lib().ee_last_kernel().decode()
        run("softmax_entropy_hot", lambda: ee.softmax_entropy(logits[0], out_probs=probs[0]))
        # Context for the C0 entropy figure: the runtime's plain copy of the same
        # 8 MiB -> 8 MiB, cold; and the entropy kernel cold at config 2's
        # [4096, 14336] (234.9 MB per launch), where launch latency no longer dominates.
        rot_c = {"i": 0}

        def copy_cold():
            i = rot_c["i"] % n_rot
            rot_c["i"] += 1
            probs[i].copy_(logits[i])

        run("copy_c0_cold", copy_cold, steps=n_rot * max(1, args.steps // n_rot), warmup=n_rot)
        if not only or "softmax_entropy_c2_cold" in only:
            R2, S2 = 4096, 14336
            sc2 = torch.from_numpy(np.exp(rng.uniform(np.log(0.1), np.log(30.0), R2)).astype(np.float32))
            L2 = (torch.randn(R2, S2, generator=torch.Generator().manual_seed(2)) * sc2[:, None]).half()
            big_in = [L2.to(dev) for _ in range(3)]                  # 3 x 235 MB > 2 x MALL
            big_out = [torch.empty_like(big_in[0]) for _ in range(3)]
            rot2 = {"i": 0}

            def ent_c2():
                i = rot2["i"] % 3
                rot2["i"] += 1
                ee.softmax_entropy(big_in[i], out_probs=big_out[i])

            run("softmax_entropy_c2_cold", ent_c2, steps=3 * max(1, args.steps // 6), warmup=6)
            # the same with non-temporal logits loads forced (option se_nt = 2: faster from
            # HBM, slower on logits a producer has just written; automatic leaves them off here)
            eel.check(eel.lib().ee_engine_set_option(eel.engine(), b"se_nt", 2))
            run("softmax_entropy_c2_cold_nt", ent_c2, steps=3 * max(1, args.steps // 6), warmup=6)
            eel.check(eel.lib().ee_engine_set_option(eel.engine(), b"se_nt", 0))
            del big_in, big_out
        run("quant_i8", lambda: ee.quantize_activations(a, "dispatcher", out_codes=a_i8, out_scale=s_i8))
        run("quant_f8", lambda: ee.quantize_activations(a, "fp8", out_codes=a_f8, out_scale=s_f8))
        run("launcher_int8", lambda: ee.gemm("int8", *ee.quantize_activations(a, "dispatcher", out_codes=a_i8,
                                                                                out_scale=s_i8)[:1], pw.i8,
                                             s_i8, pw.scale, out=c), primary="eager")
        run("torch_matmul_fp16", lambda: torch.matmul(a, w16.t()), primary="eager")
        try:                                                           # vendor INT8 GEMM (hipBLASLt) comparator
            b_kn = pw.i8.t().contiguous()
            torch._int_mm(a_i8, b_kn)
            run("torch_int_mm", lambda: torch._int_mm(a_i8, b_kn), primary="eager")
        except RuntimeError as e:
            print(f"# torch._int_mm unavailable: {e}", file=sys.stderr)
        if "hbm_copy" in only:                                         # PMC calibration: 256 MiB read + 256 MiB written
            # an elementwise kernel (a device-to-device copy_ of this size goes to the DMA engine)
            src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
            dst = torch.empty_like(src)
            run("hbm_copy", lambda: torch.neg(src, out=dst))
        # ---- configs 1 and 2: the tier GEMMs at M = 4096 (several tiles per CU: the persistent
        # kernels) -- config 1 [4096, 4096, 4096] with FP8 per-tensor scaling and 0.1% outliers of
        # magnitude 20 in A; config 2 [4096, 4096, 14336]; the FP16 baseline is torch.matmul (hipBLASLt)
        big = {}
        big_names = ("c1_int8", "c1_fp8", "c1_fp8_tensor", "c1_fp16_torch", "c1_w8a16", "c2_int8", "c2_fp8",
                     "c2_fp16_torch", "c2_w8a16")
        if not only or any(n in only for n in big_names):
            for cfg, (Mb, Kb, Nb) in (("c1", (4096, 4096, 4096)), ("c2", (4096, 4096, 14336))):
                if only and not any(n.startswith(cfg) for n in only):
                    continue
                gb = torch.Generator().manual_seed(11 if cfg == "c1" else 12)
                Ab = torch.randn(Mb, Kb, generator=gb)
                if cfg == "c1":
                    hit = torch.rand(Mb, Kb, generator=gb) < 1e-3
                    Ab = torch.where(hit, 20.0 * torch.sign(torch.randn(Mb, Kb, generator=gb)), Ab)
                ab = Ab.half().to(dev)
                Wb = (torch.randn(Nb, Kb, generator=gb) * 0.02).half().to(dev)
                Bb, bsb = ee.quantize_weights_int8(Wb)
                pwb = ee.prepare_weight(Bb, bsb).materialize()
                ai_b, si_b = ee.quantize_activations(ab, "dispatcher")
                cb = torch.empty((Mb, Nb), dtype=torch.float16, device=dev)
                run(f"{cfg}_int8", lambda: ee.gemm("int8", ai_b, pwb.i8, si_b, pwb.scale, out=cb), primary="eager")
                # FP8 in the reference's scheme (kernels.py:354-373: per-row e4m3 codes of A,
                # the int8 weight codes as e4m3, per-channel scales) at both configs, and at
                # config 1 also with per-tensor amax scales of A and W
                af_b, sf_b = ee.quantize_activations(ab, "fp8")
                run(f"{cfg}_fp8", lambda: ee.gemm("fp8", af_b, pwb.f8, sf_b, pwb.scale, out=cb), primary="eager")
                if cfg == "c1":
                    ca, sa = ee.quantize_tensor_fp8(ab)
                    cw, sw = ee.quantize_tensor_fp8(Wb)
                    run("c1_fp8_tensor", lambda: ee.gemm("fp8", ca, cw, sa, sw, out=cb), primary="eager")
                run(f"{cfg}_fp16_torch", lambda: torch.matmul(ab, Wb.t(), out=cb), primary="eager")
                run(f"{cfg}_w8a16", lambda: ee.gemm("fp16", ab, pwb.f16, out=cb), primary="eager")   # own FP16 tier
                big[cfg] = 2.0 * Mb * Nb * Kb
                del ab, Wb, Bb, pwb, ai_b, cb
        # config 1's softmax + entropy: fp16 [4096, 4096] rows drawn as in config 0, with
        # probabilities, cold (9 buffer pairs of 64 MiB > 2 x the 256 MB MALL)
        if not only or "c1_softmax_entropy" in only:
            R1, S1 = 4096, 4096
            sc1 = torch.from_numpy(rng.choice(np.float32([0.25, 1.0, 4.0, 16.0]), R1))
            L1 = (torch.randn(R1, S1, generator=torch.Generator().manual_seed(4)) * sc1[:, None]).half().to(dev)
            c1_in = [L1] + [L1.clone() for _ in range(8)]
            c1_out = [torch.empty_like(L1) for _ in range(9)]
            rot1 = {"i": 0}

            def ent_c1():
                i = rot1["i"] % 9
                rot1["i"] += 1
                ee.softmax_entropy(c1_in[i], out_probs=c1_out[i])

            run("c1_softmax_entropy", ent_c1, steps=9 * max(1, args.steps // 9), warmup=9)
            # non-temporal logits loads forced (the automatic choice keeps them for logits
            # and probabilities beyond the MALL; these buffers are cold by construction)
            eel.check(eel.lib().ee_engine_set_option(eel.engine(), b"se_nt", 2))
            run("c1_softmax_entropy_nt", ent_c1, steps=9 * max(1, args.steps // 9), warmup=9)
            eel.check(eel.lib().ee_engine_set_option(eel.engine(), b"se_nt", 0))
            del c1_in, c1_out, L1
        # ---- config 3: the dispatcher end to end on a mixed batch (M = K = N = 4096)
        c3 = None
        c3_names = ("c3_entropy", "c3_route", "c3_linear", "c3_end_to_end", "c3_routed_gemm", "c3_tier_i8",
                    "c3_tier_f8", "c3_tier_f16")
        if not only or any(n in only for n in c3_names):
            M3 = K3 = N3 = 4096
            L3, _ = mixture_logits(rng, M3, K3)
            X3 = torch.from_numpy(rng.standard_normal((M3, K3), dtype=np.float32)).half()
            W3 = (torch.from_numpy(rng.standard_normal((N3, K3), dtype=np.float32)) * 0.02).half()
            l3, x3 = torch.from_numpy(L3).to(dev), X3.to(dev)
            B3, bs3 = ee.quantize_weights_int8(W3.to(dev))
            pw3 = ee.prepare_weight(B3, bs3).materialize()
            out3 = torch.empty((M3, N3), dtype=torch.float16, device=dev)
            ws3 = (torch.empty((M3, K3), dtype=torch.uint8, device=dev),
                   torch.empty(M3, dtype=torch.float32, device=dev))
            _, h3, _ = ee.softmax_entropy(l3, probs=False)
            fr = {}
            for tl, th in ((0.41, 1.68), (2.34, 6.03)):
                _, _, cnt = ee.route(h3, tl, th)
                fr[f"({tl},{th})"] = [round(v / M3, 4) for v in cnt.cpu().tolist()]
            _, idx3, counts3 = ee.route(h3, 0.41, 1.68)

            def c3_all():
                _, h, _ = ee.softmax_entropy(l3, probs=False)
                _, idx, counts = ee.route(h, 0.41, 1.68)
                ee.routed_linear(x3, pw3, idx, counts, out=out3, workspace=ws3)

            run("c3_entropy", lambda: ee.softmax_entropy(l3, probs=False))
            run("c3_route", lambda: ee.route(h3, 0.41, 1.68))
            run("c3_linear", lambda: ee.routed_linear(x3, pw3, idx3, counts3, out=out3, workspace=ws3))
            run("c3_end_to_end", c3_all)
            # the routed GEMM launch alone (on the codes its quantiser left in the workspace)
            # against the three tiers' own GEMMs on the same partitioned rows
            ee.routed_linear(x3, pw3, idx3, counts3, out=out3, workspace=ws3)
            n0, n1, n2 = counts3.cpu().tolist()
            codes3, scale3 = ws3
            x16_3 = x3[idx3[n0 + n1:].long()].contiguous()
            o_t = [torch.empty((max(n, 1), N3), dtype=torch.float16, device=dev) for n in (n0, n1, n2)]
            run("c3_routed_gemm", lambda: ee.routed_linear(x3, pw3, idx3, counts3, out=out3, quantized=(codes3, scale3)))
            if n0:
                run("c3_tier_i8", lambda: ee.gemm("int8", codes3[:n0], pw3.i8, scale3[:n0], pw3.scale, out=o_t[0]))
            if n1:
                run("c3_tier_f8", lambda: ee.gemm("fp8", codes3[n0:n0 + n1], pw3.f8, scale3[n0:n0 + n1], pw3.scale,
                                                  out=o_t[1]))
            if n2:
                run("c3_tier_f16", lambda: ee.gemm("fp16", x16_3, pw3.f16, out=o_t[2]))
            c3 = {"routing_fractions": fr, "thresholds_timed": [0.41, 1.68],
                  "ops": 2.0 * M3 * N3 * K3, "rows": [n0, n1, n2]}
        # ---- the fused MLP engine at EE/test_engine.py:10's shape (B, S, H, Inter = 1, 1024, 2048, 5632)
        mlp = None
        mlp_names = ("mlp_int8", "mlp_fp8", "mlp_fp16", "mlp_routed", "mlp_torch_fp16")
        if not only or any(n in only for n in mlp_names):
            Sm, Hm, Fm = 1024, 2048, 5632
            gm = torch.Generator().manual_seed(3)
            hid = torch.randn(1, Sm, Hm, generator=gm).half().to(dev)
            # 1/sqrt(fan_in) weights: EE/test_engine.py:12-14's unit-variance ones overflow fp16 in down_proj
            wg, wu = ((torch.randn(Fm, Hm, generator=gm) / Hm ** 0.5).half().to(dev) for _ in range(2))
            wd = (torch.randn(Hm, Fm, generator=gm) / Fm ** 0.5).half().to(dev)
            eng_m = ee.EntropyMLPEngine(wg, wu, wd, 1.5, 2.5)
            h_tok = torch.from_numpy(rng.choice(np.float32([1.0, 2.0, 3.0]), Sm, p=[0.2, 0.4, 0.4])).to(dev)
            torch.cuda.synchronize()
            run("mlp_int8", lambda: eng_m.forward(hid, 1.0), primary="eager")
            run("mlp_fp8", lambda: eng_m.forward(hid, 2.0), primary="eager")
            run("mlp_fp16", lambda: eng_m.forward(hid, 3.0), primary="eager")
            run("mlp_routed", lambda: eng_m.forward(hid, h_tok), primary="eager")

            def mlp_torch():                                           # EE/test_engine.py:33-39, one tier
                F_ = torch.nn.functional
                return F_.linear(F_.silu(F_.linear(hid, wg)) * F_.linear(hid, wu), wd)

            run("mlp_torch_fp16", mlp_torch, primary="eager")
            mlp = {"ops": 2.0 * Sm * Hm * Fm * 3}
            del eng_m
        # ---- config 4: TinyLlama-1.1B architecture, every linear entropy-gated at (2.34, 6.03)
        c4 = None
        if not only or any(n in only for n in ("c4_forward", "c4_forward_fp16")):
            model = ee.EntropyGatedLlama.random_init(ee.TINYLLAMA_1B, seed=0, tau_low=2.34, tau_high=6.03)
            g4 = torch.Generator(device=dev)
            g4.manual_seed(1)
            ids = torch.randint(0, ee.TINYLLAMA_1B["vocab"], (8, 512), generator=g4, device=dev)
            ref16 = model.forward(ids, gated=False).float()
            gated = model.forward(ids).float()
            rows = model.last_fractions.tolist()
            err = (gated - ref16).abs().max().item()
            absmax = ref16.abs().max().item()
            del gated, ref16
            # each forward issues ~450 launches: both runs are also captured once as a HIP graph and
            # replayed (routing lives on the device, so the gated forward needs no host synchronisation)
            run("c4_forward", lambda: model.forward(ids), steps=5, warmup=2, primary="graph")
            run("c4_forward_fp16", lambda: model.forward(ids, gated=False), steps=5, warmup=2, primary="graph")
            c4 = {"rows": rows, "err": err, "absmax": absmax}
            del model
    if only:
        print(json.dumps({k: v for k, v in results.items()}))
        return

    t_i8 = results["gemm_i8"]["ms"]
    tops = ops / (t_i8 * 1e-3) / 1e12
    f8_tflops = ops / (results["gemm_f8"]["ms"] * 1e-3) / 1e12
    f16_tflops = ops / (results["gemm_f16w8"]["ms"] * 1e-3) / 1e12
    ent_gbs = ent_bytes / (results["softmax_entropy_cold"]["ms"] * 1e-3) / 1e9
    ent_hot_gbs = ent_bytes / (results["softmax_entropy_hot"]["ms"] * 1e-3) / 1e9
    q_bytes = M * K * 2 + M * K + M * 4
    kernels = {
        "gemm_i8": {"us": t_i8 * 1e3, "TOPS": tops, "frac_of_peak": tops / PEAK_I8_TOPS},
        "gemm_f8": {"us": results["gemm_f8"]["ms"] * 1e3, "TFLOPS": f8_tflops, "frac_of_peak": f8_tflops / PEAK_F8_TFLOPS},
        "gemm_f16w8": {"us": results["gemm_f16w8"]["ms"] * 1e3, "TFLOPS": f16_tflops,
                       "frac_of_peak": f16_tflops / PEAK_F16_TFLOPS},
        "softmax_entropy": {"us_cold": results["softmax_entropy_cold"]["ms"] * 1e3, "GBps_cold": ent_gbs,
                            "frac_of_hbm_cold": ent_gbs / PEAK_HBM_GBS,
                            "us_hot": results["softmax_entropy_hot"]["ms"] * 1e3, "GBps_hot": ent_hot_gbs,
                            "bytes_per_launch": ent_bytes},
        "copy_c0_cold": {"us": results["copy_c0_cold"]["ms"] * 1e3,
                         "GBps": ER * ES * 4 / (results["copy_c0_cold"]["ms"] * 1e-3) / 1e9,
                         "note": "runtime copy of the entropy kernel's bytes at C0, cold"},
        "softmax_entropy_c2": {"us_cold": results["softmax_entropy_c2_cold"]["ms"] * 1e3,
                               "GBps_cold": (4096 * 14336 * 4 + 4096 * 4)
                               / (results["softmax_entropy_c2_cold"]["ms"] * 1e-3) / 1e9,
                               "frac_of_hbm_cold": (4096 * 14336 * 4 + 4096 * 4)
                               / (results["softmax_entropy_c2_cold"]["ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS,
                               "shape": "config 2: fp16 [4096, 14336], row scales log-uniform in [0.1, 30]",
                               "us_cold_nt_loads": results["softmax_entropy_c2_cold_nt"]["ms"] * 1e3
                               if "softmax_entropy_c2_cold_nt" in results else None},
        "quant_i8": {"us": results["quant_i8"]["ms"] * 1e3,
                     "GBps": q_bytes / (results["quant_i8"]["ms"] * 1e-3) / 1e9},
        "quant_f8": {"us": results["quant_f8"]["ms"] * 1e3,
                     "GBps": q_bytes / (results["quant_f8"]["ms"] * 1e-3) / 1e9},
        "launcher_int8_eager": {"us": results["launcher_int8"]["ms"] * 1e3,
                                "TOPS": ops / (results["launcher_int8"]["ms"] * 1e-3) / 1e12},
        "torch_matmul_fp16": {"us": results["torch_matmul_fp16"]["ms"] * 1e3,
                              "TFLOPS": ops / (results["torch_matmul_fp16"]["ms"] * 1e-3) / 1e12},
        "torch_int_mm_hipblaslt": ({"us": results["torch_int_mm"]["ms"] * 1e3,
                                    "TOPS": ops / (results["torch_int_mm"]["ms"] * 1e-3) / 1e12}
                                   if "torch_int_mm" in results else None),
    }
    if c3 is not None:
        kernels["dispatcher_c3"] = {
            "us_end_to_end": results["c3_end_to_end"]["ms"] * 1e3,
            "us_entropy": results["c3_entropy"]["ms"] * 1e3,
            "us_route": results["c3_route"]["ms"] * 1e3,
            "us_routed_linear": results["c3_linear"]["ms"] * 1e3,
            "TOPS_routed_linear": c3["ops"] / (results["c3_linear"]["ms"] * 1e-3) / 1e12,
            "routing_fractions_int8_fp8_fp16": c3["routing_fractions"],
            "shape": "M=K=N=4096; entropy over fp16 [4096,4096] mixture logits",
        }
        if "c3_routed_gemm" in results:
            tiers = [results[f"c3_tier_{t}"]["ms"] * 1e3 for t in ("i8", "f8", "f16") if f"c3_tier_{t}" in results]
            kernels["dispatcher_c3"].update({
                "us_routed_gemm": results["c3_routed_gemm"]["ms"] * 1e3,
                "us_per_tier_gemms": tiers, "us_per_tier_gemm_sum": sum(tiers),
                "routed_over_per_tier_sum": results["c3_routed_gemm"]["ms"] * 1e3 / sum(tiers),
                "rows_per_tier": c3["rows"],
                "note": "routed GEMM launch alone (codes from its quantiser) vs the three tiers' own GEMMs on the "
                        "same partitioned rows, each a separate launch"})
    for cfg, ops_b in big.items():
        legs = ("int8", "fp8", "fp8_tensor", "w8a16", "fp16_torch") if cfg == "c1" else ("int8", "fp8", "w8a16",
                                                                                          "fp16_torch")
        peak = {"int8": PEAK_I8_TOPS, "fp8_tensor": PEAK_F8_TFLOPS, "fp8": PEAK_F8_TFLOPS, "w8a16": PEAK_F16_TFLOPS,
                "fp16_torch": PEAK_F16_TFLOPS}
        kernels[f"gemm_{cfg}"] = {
            leg: {"us": results[f"{cfg}_{leg}"]["ms"] * 1e3,
                  "TOPS": ops_b / (results[f"{cfg}_{leg}"]["ms"] * 1e-3) / 1e12,
                  "frac_of_peak": ops_b / (results[f"{cfg}_{leg}"]["ms"] * 1e-3) / 1e12 / peak[leg]}
            for leg in legs}
        kernels[f"gemm_{cfg}"]["shape"] = ("M, K, N = 4096, 4096, 4096; A with 0.1% outliers of 20; fp8 = the "
                                           "reference's per-row e4m3 scheme, fp8_tensor = per-tensor amax scales; "
                                           "w8a16 = this build's FP16 tier (fp16 A, W8A16 weights)"
                                           if cfg == "c1" else "M, K, N = 4096, 4096, 14336; w8a16 = this build's "
                                           "FP16 tier")
    if "c1_softmax_entropy" in results:
        b1 = 4096 * 4096 * 4 + 4096 * 4
        g1 = b1 / (results["c1_softmax_entropy"]["ms"] * 1e-3) / 1e9
        kernels["softmax_entropy_c1"] = {"us_cold": results["c1_softmax_entropy"]["ms"] * 1e3, "GBps_cold": g1,
                                         "frac_of_hbm_cold": g1 / PEAK_HBM_GBS, "bytes_per_launch": b1,
                                         "us_cold_nt_loads": results["c1_softmax_entropy_nt"]["ms"] * 1e3
                                         if "c1_softmax_entropy_nt" in results else None,
                                         "shape": "config 1: fp16 [4096, 4096] with probabilities, rows as config 0"}
    if mlp is not None:
        kernels["mlp_engine"] = {
            f"us_{k}": results[f"mlp_{k}"]["ms"] * 1e3 for k in ("int8", "fp8", "fp16", "routed", "torch_fp16")}
        kernels["mlp_engine"].update({
            f"TOPS_{k}": mlp["ops"] / (results[f"mlp_{k}"]["ms"] * 1e-3) / 1e12
            for k in ("int8", "fp8", "fp16", "routed", "torch_fp16")})
        kernels["mlp_engine"]["shape"] = ("EntropyMLPEngine.forward, B, S, H, Inter = 1, 1024, 2048, 5632 "
                                          "(EE/test_engine.py:10); routed = per-token tiers 20/40/40 %; "
                                          "torch_fp16 = the test's F.linear chain on the fp16 weights (hipBLASLt)")
    if c4 is not None:
        tot = sum(c4["rows"])
        kernels["llama_c4"] = {
            "ms_forward_gated": results["c4_forward"]["ms"],
            "ms_forward_all_fp16": results["c4_forward_fp16"]["ms"],
            "timing": "HIP graph replay of the captured forward (eager-launch figures in timings_us)",
            "routing_fraction_int8_fp8_fp16": [round(r / tot, 4) for r in c4["rows"]],
            "max_abs_logit_err_vs_fp16": c4["err"],
            "logit_absmax_fp16": c4["absmax"],
            "shape": "TinyLlama-1.1B architecture (22 layers, hidden 2048, 32 Q / 4 KV heads, FFN 5632, vocab "
                     "32000), random N(0,0.02) weights, batch 8 x seq 512 uniform token ids; every linear "
                     "routed per token row at (2.34, 6.03); all-FP16 run = hipBLASLt fp16 on the original weights",
        }
    for k, r in results.items():                                       # both timings of every kernel, in us
        kernels.setdefault("timings_us", {})[k] = {
            "eager": r["ms_eager"] * 1e3, "graph": None if r["ms_graph"] is None else r["ms_graph"] * 1e3,
            "reported": r["timing"]}

    # per-launch durations of the two roofline kernels (median over K launches)
    with torch.cuda.stream(stream):
        i8_launch_ms = time_launches(lambda: ee.gemm("int8", a_i8, pw.i8, s_i8, pw.scale, out=c), args.steps,
                                     args.warmup, stream)
        rot_l = {"i": 0}

        def ent_one():
            i = rot_l["i"] % n_rot
            rot_l["i"] += 1
            ee.softmax_entropy(logits[i], out_probs=probs[i])

        ent_launch_ms = time_launches(ent_one, n_rot * max(1, args.steps // n_rot), n_rot, stream)
    # The roofline figures divide by the average launch duration over the timed
    # region of one replayed HIP graph of K launches (events on the launch
    # stream), the basis rocprofv3's per-dispatch durations agree with; the eager
    # figure is reported beside it (us_per_launch_eager).  Without graphs
    # (--no-graph) the eager figure is the basis.  The events bracketing each
    # launch separately inflate a 7 us kernel by several us, so they are kept for
    # reference only.
    def roof_ms(name):
        r = results[name]
        return r["ms_graph"] if r["ms_graph"] else r["ms_eager"]

    i8_roof_ms = roof_ms("gemm_i8")
    ent_roof_ms = roof_ms("softmax_entropy_cold")
    i8_launch_tops = ops / (i8_roof_ms * 1e-3) / 1e12
    ent_launch_gbs = ent_bytes / (ent_roof_ms * 1e-3) / 1e9
    kernels["gemm_i8"]["us_per_launch_events"] = i8_launch_ms * 1e3
    kernels["softmax_entropy"]["us_cold_per_launch_events"] = ent_launch_ms * 1e3

    # HBM-side bytes per launch from the committed FETCH_SIZE / WRITE_SIZE passes
    # (calibrated against a 256 MiB copy); null when that summary is absent.
    traffic = ent_traffic = None
    pmc = os.path.join(ROOT, "profiles", "gemm_i8_c0_hbm_traffic.txt")
    if os.path.exists(pmc):
        for line in open(pmc):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = float(line.split(":", 1)[1])
            elif line.startswith("traffic_bytes_per_launch.eek_softmax_entropy:"):
                ent_traffic = float(line.split(":", 1)[1])

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(A.numpy(), W.numpy(), L.numpy())

    line = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t_i8,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded numpy: activations N(0,1), weights N(0,0.02), logits N(0,s))",
        "config": {"workload": "config0: INT8 tier GEMM M=1024 K=4096 N=4096 (per-row/per-channel int8, int32 "
                               "accumulate, fp16 dequant); FP8 e4m3 GEMM and fused softmax+entropy fp16 "
                               "[1024,4096] in 'kernels'",
                   "M": M, "K": K, "N": N, "entropy_rows": ER, "entropy_cols": ES},
        "value_timing": "eager launches back to back, events on the launch stream (the reference's loop)",
        "roofline": {"bound": "mfma", "achieved": round(i8_launch_tops, 2), "peak": PEAK_I8_TOPS, "unit": "TOPS",
                     "timing": "average launch over the replay of one HIP graph of K back-to-back launches",
                     "frac": round(i8_launch_tops / PEAK_I8_TOPS, 4), "traffic": traffic,
                     "kernel": f"{i8_kernel} (INT8, 1024x4096x4096)", "us_per_launch": round(i8_roof_ms * 1e3, 3),
                     "us_per_launch_eager": round(results["gemm_i8"]["ms_eager"] * 1e3, 3)},
        "roofline_entropy": {"bound": "hbm", "achieved": round(ent_launch_gbs, 1), "peak": PEAK_HBM_GBS,
                             "unit": "GB/s", "timing": "average launch over the replay of one HIP graph of K back-to-back launches, cold",
                             "frac": round(ent_launch_gbs / PEAK_HBM_GBS, 4), "traffic": ent_traffic,
                             "kernel": f"{ent_kernel} (cold, [1024,4096])", "us_per_launch": round(ent_roof_ms * 1e3, 3),
                             "us_per_launch_eager": round(results["softmax_entropy_cold"]["ms_eager"] * 1e3, 3)},
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def cpu_threads():
    """(threads, affinity, quota): the CPUs this process may run on
    (len(os.sched_getaffinity(0))), capped by the cgroup CPU quota when one is
    set (the GPU box grants each GPU a share of a larger host)."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    return (min(aff, quota) if quota else aff), aff, quota


def cpu_model():
    try:
        return [l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")][0]
    except (OSError, IndexError):
        return "unknown"


def cpu_baseline(A, W, L):
    """The reference path's arithmetic on this host's cores, on the config-0
    workload, as PyTorch's CPU ops run it: oracle/torch_cpu.py --
    INT8 = the dispatcher quantiser + torch._int_mm + epilogue (`value`), FP8 =
    e4m3 codes decoded to f32 + an f32 matmul, softmax+entropy in f32, each at
    the full 1024x4096x4096 / [1024, 4096] shape -- and the repository's C
    oracle (OpenMP) on the INT8 path beside it.  torch.set_num_threads(the
    process's CPUs); time.perf_counter around each call, 3 warmup calls, then
    the median of 10."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    import oracle
    from oracle import torch_cpu as tc
    threads, affinity, quota = cpu_threads()
    torch.set_num_threads(threads)

    def median_s(fn, warm=3, reps=10):
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        ts.sort()
        return 0.5 * (ts[reps // 2 - 1] + ts[reps // 2])

    a, w, lg = torch.from_numpy(A), torch.from_numpy(W), torch.from_numpy(L)
    B, bs = oracle.quantize_weights_int8(W)
    b, bst = torch.from_numpy(B), torch.from_numpy(bs)
    ops = 2.0 * M * N * K
    t_i8 = median_s(lambda: tc.triton_int8_gemm(a, b, bst))
    b8 = tc.weight_f8(b)
    t_f8 = median_s(lambda: tc.triton_fp8_gemm(a, b, bst, b8))
    t_e = median_s(lambda: tc.softmax_entropy(lg))
    ent_b = ER * ES * 4 + ER * 4

    def c_int8():
        codes, s = oracle.quant_act_i8(A, "dispatcher")
        return oracle.epilogue_i8(oracle.gemm_i8_acc(codes, B), s, bs)

    t_c = median_s(c_int8, warm=1, reps=4)
    model = cpu_model()
    return {"value": round(ops / t_i8 / 1e12, 4), "unit": "TOPS", "cores": threads, "kind": "port",
            "cpu_model": model, "cpus_affinity": affinity, "cpu_quota": quota,
            "int8_tops": round(ops / t_i8 / 1e12, 4), "int8_ms": round(t_i8 * 1e3, 3),
            "fp8_tflops": round(ops / t_f8 / 1e12, 4), "fp8_ms": round(t_f8 * 1e3, 3),
            "entropy_gbps": round(ent_b / t_e / 1e9, 3), "entropy_ms": round(t_e * 1e3, 3),
            "c_oracle_int8_tops": round(ops / t_c / 1e12, 4), "c_oracle_threads": oracle.num_threads(),
            "timing": "time.perf_counter per call; 3 warmup calls, median of 10 (C oracle: 1 warmup, median of 4)",
            "sample": f"PyTorch-CPU restatement (oracle/torch_cpu.py), {threads} threads on {model}: INT8 dispatcher "
                      f"quantiser + torch._int_mm + epilogue at 1024x4096x4096 ({t_i8 * 1e3:.1f} ms); FP8 codes -> f32 "
                      f"matmul at 1024x4096x4096 ({t_f8 * 1e3:.1f} ms); f32 softmax+entropy [1024,4096] "
                      f"({t_e * 1e3:.1f} ms); C oracle INT8 path ({t_c * 1e3:.1f} ms)"}


if __name__ == "__main__":
    main()
