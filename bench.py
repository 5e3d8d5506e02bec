#!/usr/bin/env python3
"""Yv MoE layer forward on one MI355X: tokens/s, roofline fraction, CPU baseline.

A step is one forward of the whole layer (router GEMM + complexity predictor, routing,
permutation, grouped SwiGLU FFN of routed and shared experts, combine with the skip residual)
over one packed batch whose inputs and weights are already resident in HBM.

Default workload: BASELINE configs[1] (cfg2) — W8A16 layer, hidden 4096, 64 experts (FFN
1408), top-6, 2 shared experts, decode batch of 64 sequences x 1 token. The same run also
times configs[2] (cfg3, the same layer on a ~16K-token ragged prefill) as the "prefill"
object, and the CPU oracle (the reference algorithm restated in torch on the host) on cfg2
as "cpu_baseline", with bounded samples of cfg3, cfg1, cfg4 and cfg5 beside it.

roofline: the dominant kernel is the grouped expert FFN (yvmoe_expert_ffn: tile schedule,
gate/up GEMM with SwiGLU, down GEMM); its average duration is measured with HIP events on
the stream it runs on. Algorithmic bytes per launch = packed weights of the experts that
received tokens + the shared experts + x (N*H*2) + y (rows*H*2); algorithmic FLOPs =
6*H*F*(N*k + N*S).

roofline.traffic: HBM bytes per launch of the same kernel, from two rocprofv3 counter runs of
``bench.py --pmc-probe cfg2`` (FETCH_SIZE, then WRITE_SIZE), each scaled by what the counter
reads for the probe's calibration copy of known size; the measured figures are kept in
profiles/expert_ffn_cfg2_decode_traffic.json and reported when present.

"moegate": the same layer shape with YvMoEGate, the router the reference's MoE layers build
(model/moe/layer.py:754-777): the gate alone and the layer with it, at decode and prefill.

"rmsnorm": the MoE input norms of the hybrid block (two RMSNorms in one pass) at the decode
and prefill token counts, HBM roofline of the kernel.

"other_configs": configs[0], [3], [4] (cfg1 fp32, cfg4 W4A16 mixed batch, cfg5 fp8 with skewed
routing): layer step and grouped FFN, the FFN against both rooflines; cfg5 also reports its
realised expert load against the Zipf(1.2) target (KL).

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
       python bench.py --pmc-probe {cfg2,cfg3,cfg5,moegate,moegate_decode}   (launches only, for counter runs)
"""
import argparse
import dataclasses
import itertools
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE layer tokens/s at 1 GPU; HBM GB/s (decode) & MFMA util % (prefill)"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "expert_ffn_cfg2_decode_traffic.json")
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_PEAK_TFLOPS = 157.3


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--no-moegate", action="store_true",
                    help="skip the YvMoEGate router and the layer built with it")
    ap.add_argument("--no-norm", action="store_true", help="skip the MoE input RMSNorm timing")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip cfg1 / cfg4 / cfg5 (layer step and FFN against both rooflines)")
    ap.add_argument("--pmc-probe", choices=["cfg2", "cfg3", "cfg5", "moegate", "moegate_decode"], default=None,
                    help="run the calibration copy and 5 expert-FFN launches (moegate: 3 YvMoEGate "
                         "prefill gate calls), nothing timed")
    return ap.parse_args()


def pmc_probe(name):
    """Launches for counter collection: a calibration op that reads and writes exactly 256 MiB
    (int32 bitwise_not), then five yvmoe_expert_ffn launches of the workload."""
    import torch
    from pisceslx_amd import functional as yvf
    from pisceslx_amd.workloads import make_workload, mix_weights, router_state
    n = 256 * 1024 * 1024 // 4
    src = torch.arange(n, device="cuda", dtype=torch.int32)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    if name in ("moegate", "moegate_decode"):  # the prefill / decode gate call of "moegate"
        import dataclasses
        from pisceslx_amd import _lib
        from pisceslx_amd.gate import YvMoEGate
        from pisceslx_amd.workloads import SPECS, seq_lengths
        spec = SPECS["cfg2"]
        decode = name == "moegate_decode"
        N = 64 if decode else sum(seq_lengths("cfg3", 0))
        torch.manual_seed(0)
        g = YvMoEGate(spec.hidden, spec.num_experts, top_k=spec.top_k, device="cuda",
                      dtype=torch.bfloat16).eval()
        x = torch.randn(N, spec.hidden, device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(3)).to(torch.bfloat16)
        st0 = g.gate_state(_lib.ACT_BF16, 1 if decode else N)
        # decode: three copies of the projection operand in turn, as the timed bench does, so
        # the 256 MB Infinity Cache does not serve one call's weights from the call before
        states = [st0] + ([dataclasses.replace(st0, w_proj=st0.w_proj.clone()) for _ in range(2)]
                          if decode else [])
        ws = torch.empty(1 << 31, dtype=torch.uint8, device="cuda")
        for i in range(6 if decode else 3):
            yvf.moegate_forward(x, states[i % len(states)], spec.top_k, workspace=ws)
        torch.cuda.synchronize()
        print(f"pmc probe {name}: done", flush=True)
        return
    w = make_workload(name, device="cuda", seed=0)
    st = router_state(w)
    ws = torch.empty(yvf.workspace_bytes(w.n_tokens, 1, st, w.experts), dtype=torch.uint8, device="cuda")
    routing = yvf.moe_forward(w.x, st, w.experts, mix_weights(w), None, workspace=ws)[2]
    for _ in range(5):
        yvf.expert_ffn(w.x, w.experts, routing, w.spec.top_k, workspace=ws)
    torch.cuda.synchronize()
    print(f"pmc probe {name}: done", flush=True)


def measured_traffic():
    """HBM bytes per expert-FFN launch at cfg2 from the committed counter summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            d = json.load(f)
        return int(d["hbm_bytes_per_launch"]) if d.get("workload") == "cfg2" else None
    except (OSError, ValueError, KeyError):
        return None


def steady_state(fn, min_gpu_s=0.2, window=10, tol=0.02, max_windows=200):
    """Warm-up by GPU time, not by call count: run windows of `window` calls (HIP events on
    the current stream) until at least `min_gpu_s` of GPU work has run and two consecutive
    windows agree within `tol`. A fresh GPU needs its clocks and power state to settle, which
    a few calls do not give. Returns the last window's mean per call (seconds)."""
    import torch
    stream = torch.cuda.current_stream()
    total, prev, cur = 0.0, None, None
    for _ in range(max_windows):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(window):
            fn()
        b.record(stream)
        b.synchronize()
        dt = a.elapsed_time(b) / 1e3
        total += dt
        cur = dt / window
        if total >= min_gpu_s and prev is not None and abs(cur - prev) <= tol * prev:
            break
        prev = cur
    return cur


def time_layer(yvf, x, st, experts, mix, skip, ws, steps, warmup):
    """Mean layer step: `warmup` calls, a warm-up to steady state by GPU time, then exactly
    `steps` calls bracketed by device synchronizations (host clock)."""
    import torch
    fn = lambda: yvf.moe_forward(x, st, experts, mix, skip, workspace=ws)
    for _ in range(warmup):
        fn()
    steady_state(fn)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def time_ffn(yvf, x, st, experts, mix, skip, ws, k, steps):
    """Average duration of the grouped expert FFN, HIP events on its stream, after a warm-up
    to steady state."""
    import torch
    out, shared, routing = yvf.moe_forward(x, st, experts, mix, skip, workspace=ws)
    stream = torch.cuda.current_stream()
    fn = lambda: yvf.expert_ffn(x, experts, routing, k, workspace=ws)
    steady_state(fn)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / 1e3 / steps, routing


def ffn_work(spec, n_tokens, routing):
    from pisceslx_amd.workloads import weight_bytes_per_expert
    active = int((routing.counts > 0).sum().item())
    rows = n_tokens * (spec.top_k + spec.num_shared)
    wbytes = (active + spec.num_shared) * weight_bytes_per_expert(spec)
    nbytes = wbytes + n_tokens * spec.hidden * 2 + rows * spec.hidden * 2
    flops = 6 * spec.hidden * spec.ffn * rows
    return {"bytes": nbytes, "weight_bytes": wbytes, "flops": flops, "active_experts": active}


def time_calls(fn, steps, warmup):
    """Average duration of fn() over `steps` calls, HIP events on the current stream."""
    import torch
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / 1e3 / steps


def moegate_bench(w, mix, steps, prefill_steps, lengths):
    """YvMoEGate (the router the reference's MoE layers build) at the cfg2 layer shape: the
    gate alone (logits, loss and routing, yvmoe_moegate_forward) at decode and prefill, and
    the layer with it as router (yvmoe_forward_moegate). Random module initialisation
    (seeded), synthetic x."""
    import torch
    from pisceslx_amd import _lib
    from pisceslx_amd import functional as yvf
    from pisceslx_amd.gate import YvMoEGate
    spec = w.spec
    H, E, k = spec.hidden, spec.num_experts, spec.top_k
    dev = w.x.device
    torch.manual_seed(0)
    g = YvMoEGate(H, E, top_k=k, device=dev, dtype=torch.bfloat16).eval()
    res = {"workload": "cfg2 layer shape (hidden 4096, 64 experts, top-6), YvMoEGate router with "
                       "all four auxiliary heads, random seeded weights"}
    for name, N, n_steps in (("decode", w.n_tokens, steps), ("prefill", sum(lengths), prefill_steps)):
        gen = torch.Generator(device=dev).manual_seed(3)
        x = torch.randn(N, H, device=dev, generator=gen).to(torch.bfloat16)
        seq = 1 if name == "decode" else N  # decode: B x 1 tokens; prefill: one packed sequence
        st0 = g.gate_state(_lib.ACT_BF16, seq)
        P = st0.w_proj.shape[0]
        # three copies of the 138 MB projection operand, used in turn, so the 256 MB Infinity
        # Cache cannot serve the weights of one call from the call before
        states = [st0] + [dataclasses.replace(st0, w_proj=st0.w_proj.clone()) for _ in range(2)]
        ws = torch.empty(max(256, int(_lib.lib().yvmoe_forward_moegate_workspace_bytes(
            N, _lib.ACT_BF16, k, __import__("ctypes").byref(st0.struct()),
            __import__("ctypes").byref(w.experts.struct())))), dtype=torch.uint8, device=dev)
        turn = itertools.cycle(range(3))
        t_gate = time_calls(lambda: yvf.moegate_forward(x, states[next(turn)], k, workspace=ws),
                            n_steps, 3)
        t_layer = time_calls(lambda: yvf.moe_forward_moegate(x, states[next(turn)], k, w.experts,
                                                              mix, None, workspace=ws), n_steps, 3)
        del states
        wbytes = P * H * 2
        entry = {"tokens": N, "gate_ms_per_call": round(t_gate * 1e3, 4),
                 "gate_tokens_per_s": round(N / t_gate, 1),
                 "layer_ms_per_step": round(t_layer * 1e3, 4),
                 "layer_tokens_per_s": round(N / t_layer, 1),
                 "projection_rows": P}
        if name == "decode":
            nbytes = wbytes + N * H * 2 + H * 4 * 4 + N * E * 4
            achieved = nbytes / t_gate / 1e9
            entry["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                                 "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                                 "kernel": "whole yvmoe_moegate_forward call (projection GEMM, "
                                           "per-token kernel, loss, routing)",
                                 "algorithmic_bytes": nbytes}
        else:
            flops = 2 * N * H * P
            tf = flops / t_gate / 1e12
            entry["roofline"] = {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
                                 "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                 "kernel": "whole yvmoe_moegate_forward call (projection GEMM, "
                                           "per-token kernel, loss, routing)",
                                 "algorithmic_flops": flops}
        res[name] = entry
        del x, ws
    return res


def norm_bench(w, steps, lengths):
    """The MoE input norms of the hybrid block (norm_fusion then norm_mlp, one yvmoe_rmsnorm
    pass) at hidden 4096, decode and prefill token counts. Launches are captured in a HIP
    graph of `reps` kernels so the per-kernel time excludes Python's launch cost; the roofline
    prices one launch at its algorithmic bytes: x read once, y written once, two weights."""
    import torch
    from pisceslx_amd import functional as yvf
    H = w.spec.hidden
    dev = w.x.device
    gen = torch.Generator(device=dev).manual_seed(5)
    wts = [(1.0 + 0.1 * torch.randn(H, device=dev, generator=gen)).to(torch.bfloat16) for _ in range(2)]
    norms = [(wt, None, 1e-6) for wt in wts]
    res = {"workload": "two RMSNorms in sequence (YvHybridBlock norm_fusion, norm_mlp), hidden 4096, "
                       "bf16, one pass"}
    for name, N in (("decode", w.n_tokens), ("prefill", sum(lengths))):
        # three input/output pairs used in turn: at prefill one pair is 274 MB, so the 256 MB
        # Infinity Cache cannot hold the previous launch's rows
        xs = [torch.randn(N, H, device=dev, generator=gen).to(torch.bfloat16) for _ in range(3)]
        ys = [torch.empty_like(xs[0]) for _ in range(3)]
        reps = 51
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            yvf.rms_norm(xs[0], norms, out=ys[0])  # warm the launch path outside the capture
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(reps):
                yvf.rms_norm(xs[i % 3], norms, out=ys[i % 3])
        t = time_calls(graph.replay, max(3, steps // 10), 2) / reps
        nbytes = 2 * N * H * 2 + 2 * H * 2
        achieved = nbytes / t / 1e9
        res[name] = {"tokens": N, "us_per_call": round(t * 1e6, 3),
                     "timing": "HIP graph of 51 launches over three buffer pairs in turn, per node "
                               "(includes the graph's per-node launch cost, which dominates a "
                               "kernel of a few us)",
                     "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                                  "kernel": "rmsnorm_kernel (2 norms)", "algorithmic_bytes": nbytes}}
        del graph, xs, ys
    return res


def other_configs(names, steps):
    """The BASELINE configs that are not bench lines (cfg1 fp32 parity layer, cfg4 W4A16 mixed
    batch, cfg5 fp8 skewed routing): the layer step and the grouped FFN, each FFN priced against
    both rooflines (algorithmic bytes over 8 TB/s, algorithmic FLOPs over the MFMA peak of the
    compute dtype: fp32 157.3 TFLOP/s for cfg1, bf16 2.5 PFLOP/s otherwise)."""
    import torch
    from pisceslx_amd import functional as yvf
    from pisceslx_amd.quant import FORMAT_NAMES
    from pisceslx_amd.workloads import load_kl, make_workload, mix_weights, router_state, zipf_target
    res = {}
    for name in names:
        w = make_workload(name, device="cuda")
        spec = w.spec
        st, mix = router_state(w), mix_weights(w)
        act = yvf._act(spec.act_dtype)
        ws = torch.empty(yvf.workspace_bytes(w.n_tokens, act, st, w.experts), dtype=torch.uint8,
                         device=w.x.device)
        t = time_layer(yvf, w.x, st, w.experts, mix, None, ws, steps, 3)
        tf, rt = time_ffn(yvf, w.x, st, w.experts, mix, None, ws, spec.top_k, steps)
        wk = ffn_work(spec, w.n_tokens, rt)
        peak = F32_PEAK_TFLOPS if spec.act_dtype == torch.float32 else BF16_PEAK_TFLOPS
        res[name] = {"tokens": w.n_tokens, "ms_per_step": round(t * 1e3, 4),
                     "tokens_per_s": round(w.n_tokens / t, 1), "ffn_ms_per_launch": round(tf * 1e3, 4),
                     "ffn_tflops": round(wk["flops"] / tf / 1e12, 1),
                     "ffn_mfma_frac": round(wk["flops"] / tf / 1e12 / peak, 4),
                     "ffn_gbs": round(wk["bytes"] / tf / 1e9, 1),
                     "ffn_hbm_frac": round(wk["bytes"] / tf / 1e9 / HBM_PEAK_GBS, 4),
                     "active_experts": wk["active_experts"], "weights": FORMAT_NAMES[spec.fmt]}
        if spec.zipf_s > 0:
            counts = rt.counts.cpu().numpy()
            target = zipf_target(spec.num_experts, spec.zipf_s, spec.zero_experts, 0)
            res[name]["load"] = {
                "zipf_s": spec.zipf_s, "bias_beta": spec.zipf_beta,
                "kl_vs_zipf_nats": round(load_kl(counts, target), 4),
                "experts_without_tokens": int((counts == 0).sum()),
                "max_slots_per_expert": int(counts.max()),
                "note": "KL(realised || Zipf) of the slot counts; beta minimises it "
                        "(workloads.zipf_beta_search); top-8 caps an expert at one slot per "
                        "token, below the heaviest Zipf shares"}
        del w, ws
        torch.cuda.empty_cache()
    return res


def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_time(fn, budget_s, warmup=True, runs=3):
    """1 warm-up (unless warmup is False), then the median of up to `runs` timed runs within
    budget_s."""
    times = []
    t_start = time.perf_counter()
    if warmup:
        fn()
    for _ in range(runs):
        if time.perf_counter() - t_start > budget_s and times:
            break
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


# CPU baseline samples of the configurations that are not the bench line: (tokens timed,
# warm-up, timed runs). cfg1 whole; cfg4 its first two 512-token prefill chunks; cfg5 the first
# 2048 tokens, one timed run (about 10 s on 16 EPYC cores).
CPU_SAMPLES = {"cfg1": (None, True, 3), "cfg4": (1024, True, 3), "cfg5": (2048, False, 1)}


def cpu_baseline(w, x3=None, others=(), budget_s=30.0):
    """The CPU oracle (the reference algorithm restated with torch on the host: router and
    routing, per-expert loop with experts dequantized inside it, F.linear of the layer dtype as
    the reference runs it, shared experts, combine) on every core this process may use,
    bounded. The cfg2 decode batch is timed whole; for cfg3 (prefill) a leading slice of the
    packed batch is timed (the per-token cost of the full 16K-token forward, which would take
    minutes); `others` names configurations sampled as CPU_SAMPLES says (a slice is routed as a
    batch of its own: capacity from its own token count)."""
    import torch
    from oracle import moe_oracle
    from pisceslx_amd.workloads import make_workload
    cores = max(1, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    params = moe_oracle.params_from_workload(w)
    x = w.x.cpu()
    t, n = _cpu_time(lambda: moe_oracle.layer_forward(x, params, reference_linear=True), budget_s)
    res = {"value": round(w.n_tokens / t, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
           "cpu": cpu_model_name(),
           "sample": f"{w.spec.name} full forward, {w.n_tokens} tokens, 1 warm-up + median of "
                     f"{n} runs ({t:.3f} s each), experts dequantized inside the loop, "
                     f"bf16 F.linear as the reference runs it, {cores} threads"}
    if x3 is not None:
        n_tok = x3.shape[0]
        t3, n3 = _cpu_time(lambda: moe_oracle.layer_forward(x3, params, reference_linear=True),
                           budget_s)
        res["cfg3"] = {"value": round(n_tok / t3, 2), "unit": "tokens/s",
                       "sample": f"cfg3 layer on the first {n_tok} tokens of the packed prefill "
                                 f"batch, 1 warm-up + median of {n3} runs ({t3:.3f} s each)"}
    del params
    for name in others:
        n_tok, warm, runs = CPU_SAMPLES[name]
        wo = make_workload(name, device="cuda")
        po = moe_oracle.params_from_workload(wo)   # packed experts copied to host memory
        xo = (wo.x if n_tok is None else wo.x[:n_tok]).cpu()
        total = wo.n_tokens
        del wo
        torch.cuda.empty_cache()
        to, no = _cpu_time(lambda: moe_oracle.layer_forward(xo, po, reference_linear=True),
                           budget_s, warmup=warm, runs=runs)
        what = "the whole batch" if n_tok is None else f"the first {xo.shape[0]} of {total} tokens"
        res[name] = {"value": round(xo.shape[0] / to, 2), "unit": "tokens/s",
                     "sample": f"{name} layer on {what}, {'1 warm-up + ' if warm else ''}median of "
                               f"{no} run{'s' if no > 1 else ''} ({to:.3f} s each)"}
        del po, xo
    return res


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the Yv MoE layer forward runs on one MI355X "
              "here; runs over several GPUs are not part of this benchmark.", file=sys.stderr)
        sys.exit(2)
    if args.pmc_probe:
        pmc_probe(args.pmc_probe)
        return
    import torch
    from pisceslx_amd import functional as yvf
    from pisceslx_amd.workloads import make_workload, mix_weights, router_state, seq_lengths

    dev = torch.device("cuda:0")
    w = make_workload("cfg2", device=dev, seed=0)
    spec = w.spec
    st = router_state(w)
    mix = mix_weights(w)
    N, H = w.n_tokens, spec.hidden
    skip = torch.randn(N, H, device=dev, generator=torch.Generator(device=dev).manual_seed(1)).to(spec.act_dtype)
    ws = torch.empty(yvf.workspace_bytes(N, 1, st, w.experts), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    t_step = time_layer(yvf, w.x, st, w.experts, mix, skip, ws, args.steps, args.warmup)
    t_ffn, routing = time_ffn(yvf, w.x, st, w.experts, mix, skip, ws, spec.top_k, args.steps)
    work = ffn_work(spec, N, routing)
    achieved = work["bytes"] / t_ffn / 1e9
    result = {
        "metric": METRIC,
        "value": round(N / t_step, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "cfg2: W8A16 Yv MoE layer decode (BASELINE configs[1])",
                   "tokens": N, "hidden": H, "experts": spec.num_experts, "ffn": spec.ffn,
                   "top_k": spec.top_k, "shared_experts": spec.num_shared,
                   "weights": "int8 per-output-channel, bf16 scales", "seed": 0},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "kernel": "grouped expert FFN (yvmoe_expert_ffn)",
                     "ms_per_launch": round(t_ffn * 1e3, 4),
                     "algorithmic_bytes": work["bytes"], "active_experts": work["active_experts"]},
    }
    layer_bytes = work["weight_bytes"] + spec.num_experts * H * 2 + 64 * H * 4 + N * H * 2 * 4
    result["layer_hbm_gbs"] = round(layer_bytes / t_step / 1e9, 1)

    x3_cpu = None
    if not args.no_prefill:
        lengths = seq_lengths("cfg3", 0)
        Np = sum(lengths)
        gx = torch.Generator(device=dev).manual_seed(2)
        xp = torch.randn(Np, H, device=dev, generator=gx).to(spec.act_dtype)
        skip_p = torch.randn(Np, H, device=dev, generator=gx).to(spec.act_dtype)
        wsp = torch.empty(yvf.workspace_bytes(Np, 1, st, w.experts), dtype=torch.uint8, device=dev)
        tp = time_layer(yvf, xp, st, w.experts, mix, skip_p, wsp, args.prefill_steps, 3)
        tpf, rp = time_ffn(yvf, xp, st, w.experts, mix, skip_p, wsp, spec.top_k, args.prefill_steps)
        wp = ffn_work(spec, Np, rp)
        tf = wp["flops"] / tpf / 1e12
        layer_flops = wp["flops"] + 2 * Np * H * (spec.num_experts + 192)
        result["prefill"] = {
            "workload": "cfg3: same layer, ragged prefill of 32 sequences (BASELINE configs[2])",
            "tokens": Np, "tokens_per_s": round(Np / tp, 1), "ms_per_step": round(tp * 1e3, 3),
            "layer_tflops": round(layer_flops / tp / 1e12, 1),
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "kernel": "grouped expert FFN (yvmoe_expert_ffn)",
                         "ms_per_launch": round(tpf * 1e3, 4), "algorithmic_flops": wp["flops"]},
        }
        x3_cpu = xp[:1024].cpu()
        del xp, skip_p, wsp
    if not args.no_moegate:
        result["moegate"] = moegate_bench(w, mix, args.steps, args.prefill_steps, seq_lengths("cfg3", 0))
    if not args.no_norm:
        result["rmsnorm"] = norm_bench(w, args.steps, seq_lengths("cfg3", 0))
    if not args.no_other_configs:
        result["other_configs"] = other_configs(("cfg1", "cfg4", "cfg5"), max(5, args.prefill_steps // 2))
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(
            w, x3_cpu, others=() if args.no_other_configs else ("cfg1", "cfg4", "cfg5"))
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
