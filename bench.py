"""Benchmark of the MI355X MoE FFN. Default workload: BASELINE config 2, a Mixtral-8x7B-shaped MoE
layer (d 4096, 8 experts, top-2, SwiGLU d_ff 14336) with Q8_0 expert stacks and an F32 router, seeded
synthetic weights N(0, 0.02) (router N(0, 1/sqrt(d))) and hidden states N(0, 1); --config c1/c3/c4
selects the other single-layer configs.

One step = one ember_moe_ffn call over one batch of T tokens resident in HBM (the headline T is
--tokens, default the config's first = decode). Prints ONE JSON line. Besides the contract fields it
carries:
  roofline      the dominant kernel, HBM-bound (the gate/up + SwiGLU kernel; at one token with a prefill pack
                the slice kernel, which runs the router and routing, then gate/up, SwiGLU and down per
                64-column slice of d_ff): algorithmic bytes per launch over
                its average duration, timed with HIP events that the launch records in the kernel's
                own dispatch packet on the launch stream; `traffic` is the kernel's HBM bytes per launch from the
                committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary of the same workload (profiles/)
  cpu_baseline  the reference's CPU MoE path (oracle/_ref, compiled from the reference's own sources
                when present; else the oracle's restatement) on the box's host cores, on a bounded
                token sample of the same layer
  sweep         the other token counts of config 2 (µs/layer, tokens/s, roofline fractions)
  c1, c3, c4    (default c2 run) the other single-layer configs' own sweeps, same fields
  c5            (default c2 run) the end-to-end config 5 model: prefill + greedy decode tokens/s

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--config c2] [--tokens 1] [--sweep 1,8,128,2048]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "ember.cpp_amd")]

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
GRAPH_CALLS = 8              # layer calls per captured HIP graph (graph_us is per call)
MFMA_PEAK_TFLOPS = 2500.0    # dense fp16 / bf16 MFMA, the prefill kernels' operand type


def log(*a):
    print(*a, file=sys.stderr, flush=True)


CONFIGS = {
    # (description, spec kwargs, token counts)
    "c1": ("config 1: toy F32 layer, d 256, E 8, top-2, d_ff 688",
           dict(d=256, d_ff=688, E=8, k=2, wtype="f32"), [1, 64]),
    "c2": ("config 2: Mixtral-8x7B-shaped MoE layer, d 4096, E 8, top-2, d_ff 14336, Q8_0 experts",
           dict(d=4096, d_ff=14336, E=8, k=2, wtype="q8_0"), [1, 8, 128, 2048]),
    "c3": ("config 3: Qwen3-30B-A3B-shaped layer, d 2048, E 128, top-8 renorm, d_ff 768, Q4_K experts",
           dict(d=2048, d_ff=768, E=128, k=8, wtype="q4_k"), [1, 32, 4096]),
    "c4": ("config 4: DeepSeek-style layer, d 2048, 64 routed + 2 shared experts (d_ff_shared 2816), top-6, "
           "d_ff 1408, BF16 experts, seeded N(0,2) selection bias",
           dict(d=2048, d_ff=1408, E=64, k=6, wtype="bf16", bias_std=2.0, d_ff_shared=2816), [1, 2048]),
}
BPW = {"f32": 4.0, "f16": 2.0, "bf16": 2.0, "q8_0": 34.0 / 32.0, "q4_k": 144.0 / 256.0}


def layer_spec(name="c2"):
    import ember_moe as em

    kw = dict(CONFIGS[name][1])
    kw["wtype"] = em.TYPE_IDS[kw["wtype"]]
    return em.LayerSpec(seed=0, **kw)


def realised_experts(em, dl, x, T):
    """Distinct experts the batch routes to, from the product's own router and routing kernels."""
    import torch

    s = dl.host.spec
    lg = torch.empty((T, s.E), dtype=torch.float32, device="cuda")
    assert em.router_logits(x, T, s.d, s.E, dl.tensors["router"], lg) == 0
    idx = torch.empty((T, s.k), dtype=torch.int32, device="cuda")
    gates = torch.empty((T, s.k), dtype=torch.float32, device="cuda")
    offsets = torch.empty(s.E + 1, dtype=torch.int32, device="cuda")
    perm = torch.empty(T * s.k, dtype=torch.int32, device="cuda")
    scr = torch.empty(em.route_scratch_bytes(T, s.E, s.k), dtype=torch.uint8, device="cuda")
    bias = dl.tensors.get("bias")
    assert em.route(lg, T, s.E, s.k, s.renorm, s.scoring, bias, s.groups_n, s.groups_top, idx, gates, offsets, perm,
                    scr) == 0
    torch.cuda.synchronize()
    return int(np.unique(idx.cpu().numpy()).size)


def algorithmic(spec, T, U, path_bits=0):
    """Algorithmic HBM bytes of the dominant expert launch and of the whole layer (U = realised experts
    hit, shared expert included, weights counted in their ggml encoding), and the layer's flops (routed
    rows and the shared expert). The dominant launch is the gate/up + SwiGLU kernel, or, on the one-token
    slice path (path_bits & PATH_SLICES), the slice kernel: gate/up, SwiGLU and down for every pick, plus
    its partial output rows (k * d_ff / 64 rows of d floats written)."""
    import ember_moe as em

    d, dff, k, E = spec.d, spec.d_ff, spec.k, spec.E
    bpw = BPW[em.TYPE_NAMES[spec.wtype]]
    dsh = spec.d_ff_shared
    if path_bits & em.PATH_SLICES:
        gu = U * 3 * d * dff * bpw + k * (dff // 64) * d * 4 + d * 4 + E * d * 4
    else:
        gu = U * 2 * d * dff * bpw + T * k * d * 4 + T * k * dff * 4
        if T == 1:
            gu += E * d * 4  # one token: the router, routing and dispatch run inside the gate/up launch
    layer = (U * 3 * d * dff + 3 * d * dsh) * bpw + E * d * 4 + 2 * T * d * 4
    flops = 2.0 * T * (k * 3 * d * dff + 3 * d * dsh) + 2.0 * T * E * d
    return gu, layer, flops


# Consecutive calls of one layer would find part of the previous call's weights in the device's 256 MB
# last-level cache, which the layers of a model (each its own weights) do not: the timed calls cycle through
# copies of the layer, enough that a copy's weights are read again only after twice the cache's bytes.
LLC_BYTES = 256 << 20
MAX_COPIES = 16


def copies_needed(touched_bytes):
    return max(1, min(MAX_COPIES, -(-2 * LLC_BYTES // max(1, int(touched_bytes)))))


def layer_copies(dl, n, log_prefix):
    """dl and n - 1 device copies of it (DeviceLayer.clone)."""
    import torch

    dls = [dl]
    for _ in range(n - 1):
        dls.append(dl.clone())
    torch.cuda.synchronize()
    if n > 1:
        log(f"{log_prefix} timing over {n} copies of the layer")
    return dls


def run_sweep(em, spec, dl, sweep_T, steps, warmup, log_prefix="[bench]"):
    """Per token count: eager and graph timing of the layer call (cycling through copies of the layer, see
    LLC_BYTES), per-phase times and the roofline fractions; returns {T: entry}."""
    import torch

    results = {}
    xs, need = {}, 1
    for T in sweep_T:
        xs[T] = torch.from_numpy(em.make_input(spec, T)).cuda()
        U = realised_experts(em, dl, xs[T], T)
        need = max(need, copies_needed(algorithmic(spec, T, U, em.path(dl.desc, T))[1]))
    dls = layer_copies(dl, need, log_prefix)
    for T in sweep_T:
        x = xs[T]
        U = realised_experts(em, dl, x, T)
        bits = em.path(dl.desc, T)
        gu_bytes, layer_bytes, flops = algorithmic(spec, T, U, bits)
        ncop = min(len(dls), copies_needed(layer_bytes))
        eager_ms, graph_ms, phases, _ = time_layer(em, dls[:ncop], x, T, steps, warmup)
        best_ms = min(eager_ms, graph_ms) if graph_ms else eager_ms
        gu_ms = phases["gate_up"]
        results[T] = dict(T=T, experts_hit=U, path_bits=bits, layer_copies=ncop, us_per_layer=best_ms * 1e3,
                          eager_us=eager_ms * 1e3,
                          layer_mfma_frac=flops / (best_ms * 1e-3) / (MFMA_PEAK_TFLOPS * 1e12),
                          graph_us=None if graph_ms is None else graph_ms * 1e3, tokens_per_s=T / (best_ms * 1e-3),
                          layer_hbm_frac=layer_bytes / (best_ms * 1e-3) / (HBM_PEAK_GBS * 1e9),
                          gate_up_us=gu_ms * 1e3, gate_up_gbs=gu_bytes / (gu_ms * 1e-3) / 1e9,
                          gate_up_hbm_frac=gu_bytes / (gu_ms * 1e-3) / (HBM_PEAK_GBS * 1e9),
                          layer_tflops=flops / (best_ms * 1e-3) / 1e12,
                          phases_us={p: round(v * 1e3, 2) for p, v in phases.items()})
        log(f"{log_prefix} T={T}: {json.dumps(results[T])}")
    del dls
    torch.cuda.empty_cache()
    return results


def nested_config(em, name, steps, warmup):
    """Another BASELINE layer config's own sweep (its token counts), with the prefill pack where the layer
    has one, for the default run's JSON line."""
    import torch

    spec = layer_spec(name)
    t0 = time.time()
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    if em.prefill_pack_bytes(dl.desc) > 0:
        dl.tensors["pack"] = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
        em.prefill_pack(dl.desc, dl.tensors["pack"])
    torch.cuda.synchronize()
    log(f"[bench {name}] layer ready in {time.time() - t0:.1f}s")
    desc, _, tokens = CONFIGS[name]
    res = run_sweep(em, spec, dl, tokens, steps, warmup, log_prefix=f"[bench {name}]")
    out = {"workload": desc, "sweep": [res[T] for T in tokens]}
    del dl
    torch.cuda.empty_cache()
    return out


def time_layer(em, dls, x, T, steps, warmup):
    """Eager timing of K steps bracketed by synchronisations and events on the launch stream, then HIP-graph
    replays of the same calls, GRAPH_CALLS calls per graph (each replay checked bit-identical to eager).
    Call i runs on copy i % len(dls) of the layer (the same weights)."""
    import torch

    dl = dls[0]
    R = len(dls)
    out = torch.empty_like(x)
    scratch = torch.empty(em.scratch_bytes(dl.desc, T), dtype=torch.uint8, device="cuda")
    for i in range(max(warmup, R)):
        dls[i % R].forward(x, out, scratch)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        em.moe_ffn(dls[i % R].desc, x, T, out, scratch)
    e1.record(st)
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / steps
    ref_out = out.clone()

    # HIP graph: GRAPH_CALLS consecutive calls captured in one graph (as an engine's decode-step graph holds
    # every layer, so one graph launch is shared by many layer calls), replayed; per-call time. Every
    # replay's output is checked bit-identical to the eager output.
    graph_ms = None
    try:
        g = torch.cuda.CUDAGraph()
        s2 = torch.cuda.Stream()
        s2.wait_stream(st)
        with torch.cuda.stream(s2):
            em.moe_ffn(dl.desc, x, T, out, scratch)  # warm on the capture stream
        st.wait_stream(s2)
        torch.cuda.synchronize()
        ncalls = max(GRAPH_CALLS, R)
        with torch.cuda.graph(g):
            for i in range(ncalls):
                status = em.moe_ffn(dls[i % R].desc, x, T, out, scratch)
                assert status == 0
        out.zero_()
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        if not torch.equal(out.view(torch.int32), ref_out.view(torch.int32)):
            raise RuntimeError("graph replay differs from eager output")
        reps = max(1, steps // ncalls)
        e0.record(st)
        for _ in range(reps):
            g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        graph_ms = e0.elapsed_time(e1) / (reps * ncalls)
        if not torch.equal(out.view(torch.int32), ref_out.view(torch.int32)):
            raise RuntimeError("graph replay differs from eager output")
    except Exception as exc:  # the eager number stands alone
        log(f"[bench] graph capture skipped: {exc}")

    # per-phase times; on the decode path the expert phases are the kernels' own durations (events in
    # their dispatch packets), i.e. what rocprofv3 --kernel-trace reports for them
    phases = {p: 0.0 for p in em.PHASES}
    n = max(3, min(steps, 20))
    for i in range(n):
        for p, v in em.moe_ffn_timed(dls[i % R].desc, x, T, out, scratch).items():
            phases[p] += v / n
    return eager_ms, graph_ms, phases, out


def profiled_traffic(config, T):
    """HBM bytes per launch of the gate/up kernel, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary of this workload (profiles/*.md, line 'bench-traffic: <config> T=<T> gate_up <bytes>'), or
    None when no summary covers it."""
    d = os.path.join(ROOT, "profiles")
    if not os.path.isdir(d):
        return None
    key = f"bench-traffic: {config} T={T} gate_up "
    for name in sorted(os.listdir(d)):
        if name.endswith(".md"):
            with open(os.path.join(d, name)) as f:
                for ln in f:
                    if ln.startswith(key):
                        return float(ln[len(key):].split()[0])
    return None


def _host_info():
    import multiprocessing

    return {"nproc": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else multiprocessing.cpu_count(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "host_cpu": _cpu_model()}


def cpu_baseline(hl, spec, sweep_T, max_seconds=12.0, prefill_seconds=6.0):
    """The reference's CPU MoE path on the GPU box's host, on F32 stacks dequantized from the same
    encoded bytes (weight_management.cpp:802-877):
      decode  moe_ffn_f32_cpu at T = 1, single-threaded, as model.cpp:759 runs it, over a bounded
              sample of independent tokens;
      prefill the same function under cpu_batch_processor.cpp:223-231's OpenMP static schedule over the
              tokens of the batch, on every host core, for each sweep T > 8, timed on a bounded
              prefix of the batch (tokens are independent, so tokens/s scales to the whole batch)."""
    from oracle import oracle as O

    s = hl.spec
    t0 = time.time()
    R = hl.router
    G, U, D = (hl.dequantized(n) for n in ("gate", "up", "down"))
    log(f"[bench] cpu baseline: dequantized F32 stacks in {time.time() - t0:.1f}s")
    plain = s.bias_std == 0 and s.d_ff_shared == 0 and s.scoring == 0 and s.groups_n <= 1 and s.out_scale == 1.0
    use_ref = O.ref_available() and plain
    sh = {}
    if s.d_ff_shared:
        sh = dict(d_ff_sh=s.d_ff_shared, Gs=hl.dequantized("gate_sh"), Us=hl.dequantized("up_sh"),
                  Ds=hl.dequantized("down_sh"))
    info = _host_info()
    cores = info["nproc"]

    def run(x, nthreads):
        out = np.empty_like(x)
        if use_ref:
            f = O.ref().ref_moe_ffn_f32 if nthreads == 1 else None
            if f is not None:
                f(x.ctypes.data, x.shape[0], s.d, s.d_ff, s.E, s.k, R.ctypes.data, G.ctypes.data, U.ctypes.data,
                  D.ctypes.data, out.ctypes.data, int(s.renorm))
            else:
                O.ref().ref_moe_ffn_f32_omp(x.ctypes.data, x.shape[0], s.d, s.d_ff, s.E, s.k, R.ctypes.data,
                                            G.ctypes.data, U.ctypes.data, D.ctypes.data, out.ctypes.data,
                                            int(s.renorm), nthreads)
        else:
            out[:] = O.moe_layer(x, R, G, U, D, s.d_ff, s.E, s.k, renorm=s.renorm, bias=hl.bias, nthreads=nthreads,
                                 **sh)
        return out

    x1 = em_input(spec, 1024)
    done, t_start = 0, time.time()
    while done < x1.shape[0] and (time.time() - t_start) < max_seconds:
        run(np.ascontiguousarray(x1[done:done + 1]), 1)
        done += 1
    el = time.time() - t_start
    res = {"value": done / el, "unit": "tokens/s", "cores": 1, "kind": "reference" if use_ref else "port",
           "sample": f"{done} decode tokens (T=1 calls) of the same layer on F32 stacks dequantized from the "
                     f"same encoded bytes, single thread, {el:.1f}s", **info}
    prefill = []
    for T in sweep_T:
        if T <= 8:
            continue
        x = em_input(spec, T)
        # a first chunk of one token per core sizes the timed prefix to about prefill_seconds
        n = min(T, cores)
        t_s = time.time()
        run(np.ascontiguousarray(x[:n]), cores)
        per_tok = (time.time() - t_s) / n
        n = int(min(T, max(cores, cores * round(prefill_seconds / max(per_tok * cores, 1e-6)))))
        t_s = time.time()
        run(np.ascontiguousarray(x[:n]), cores)
        el = time.time() - t_s
        prefill.append({"T": T, "value": n / el, "unit": "tokens/s", "cores": cores,
                        "sample": f"the first {n} of the T={T} batch's tokens, OpenMP static over tokens on "
                                  f"{cores} threads, {el:.1f}s"})
        log(f"[bench] cpu prefill T={T}: {n / el:.1f} tokens/s ({n} tokens, {el:.1f}s, {cores} threads)")
    res["prefill"] = prefill
    return res


def em_input(spec, T):
    import ember_moe as em

    return em.make_input(spec, T)


def bench_vendor_gemm(args):
    """Times torch.matmul in fp16 with random operands (hipBLASLt / rocBLAS underneath) on the dense GEMMs a
    config's prefill layer reduces to: all T k routed rows against one expert's gate+up (N = 2 d_ff, K = d)
    and down (N = d, K = d_ff) matrices, and the per-expert share T k / E rows, plus 8192^3. A measured
    reference for what the matrix cores sustain on this box, beside the datasheet peak."""
    import torch

    desc, _, tokens = CONFIGS[args.config]
    spec = layer_spec(args.config)
    T = args.tokens or max(tokens)
    rows = T * spec.k
    shapes = [(rows, 2 * spec.d_ff, spec.d), (rows, spec.d, spec.d_ff),
              (max(1, rows // spec.E), 2 * spec.d_ff, spec.d), (max(1, rows // spec.E), spec.d, spec.d_ff),
              (8192, 8192, 8192)]
    out = []
    for M, N, K in shapes:
        a = torch.randn(M, K, device="cuda", dtype=torch.float16)
        b = torch.randn(K, N, device="cuda", dtype=torch.float16)
        for _ in range(3):
            a @ b
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            a @ b
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / args.steps * 1e3
        out.append({"M": M, "N": N, "K": K, "us": round(us, 1), "tflops": round(2 * M * N * K / us / 1e6, 1)})
        log(f"[vendor-gemm] M={M} N={N} K={K}: {us:.1f} us, {out[-1]['tflops']} TFLOP/s")
    print(json.dumps({"vendor_gemm_fp16": out, "config": args.config, "tokens": T}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=str, default="c2", choices=sorted(CONFIGS) + ["c5"])
    ap.add_argument("--tokens", type=int, default=None, help="headline token count (default: the config's first)")
    ap.add_argument("--sweep", type=str, default=None, help="comma-separated token counts (default: the config's)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-c5", action="store_true", help="skip the end-to-end config 5 run the default c2 run adds")
    ap.add_argument("--no-nested", action="store_true", help="skip the config 1 / 3 / 4 sweeps the default c2 run adds")
    ap.add_argument("--no-pack", action="store_true",
                    help="run prefill without the prefill pack (Q8_0 / Q4_K tiles, BF16 row exponents)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device-to-device copies of MIB MiB (the reference kernel that scales "
                         "rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes), then exit")
    ap.add_argument("--expert-type", type=str, default=None, choices=sorted(BPW),
                    help="single-layer configs only: encode the experts in this type instead of the config's "
                         "(e.g. a Mixtral-shaped Q4_K layer, config 5's FFN, for counter passes)")
    ap.add_argument("--decode-steps", type=int, default=256,
                    help="--config c5 only: greedy decode steps after the 512-token prefill (a shorter run for "
                         "counter passes)")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only time torch's fp16 matmul (the vendor GEMM library) on the dense shapes of the config's "
                         "prefill expert GEMMs at the headline token count, as a measured ceiling, then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): the multi-GPU layout (tensor parallel "
              f"decode, expert parallel prefill) is designed, not built or measured.", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copied {args.calibrate_copy} MiB x 5")
        return

    if args.vendor_gemm:
        return bench_vendor_gemm(args)

    import ember_moe as em

    em.lib()
    if args.config == "c5":
        return bench_e2e(args)
    if args.expert_type:
        d0, kw0, tk0 = CONFIGS[args.config]
        CONFIGS[args.config] = (f"{d0.rsplit(',', 1)[0]}, experts re-encoded as {args.expert_type}",
                                dict(kw0, wtype=args.expert_type), tk0)
    desc, _, tokens = CONFIGS[args.config]
    if args.tokens is None:
        args.tokens = tokens[0]
    if args.sweep is None:
        args.sweep = ",".join(str(t) for t in tokens)
    spec = layer_spec(args.config)
    t0 = time.time()
    hl = em.make_host_layer(spec)
    log(f"[bench] generated + quantized the layer in {time.time() - t0:.1f}s")
    dl = em.DeviceLayer.upload(hl)
    # the prefill pack (tile-contiguous copy of the Q8_0 stacks for the 256-token-tile GEMM), prepared
    # once at load as a model loader would; decode does not read it
    packed = False
    if not args.no_pack and em.prefill_pack_bytes(dl.desc) > 0:
        dl.tensors["pack"] = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
        em.prefill_pack(dl.desc, dl.tensors["pack"])
        packed = True
        log(f"[bench] prefill pack: {dl.tensors['pack'].numel() / 1e9:.2f} GB")
    torch.cuda.synchronize()

    sweep_T = sorted(set([args.tokens] + [int(t) for t in args.sweep.split(",") if t]))
    results = run_sweep(em, spec, dl, sweep_T, args.steps, args.warmup)

    h = results[args.tokens]
    # the committed traffic summaries are keyed by workload: a re-encoded layer is not the config's own
    traffic_key = args.config + (f":{args.expert_type}" if args.expert_type else "")
    line = {
        "metric": "MoE-FFN tokens/s (" + args.config + ")",
        "value": h["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["us_per_layer"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{em.TYPE_NAMES[spec.wtype]} weights; decode: int16-quantized activations, int32/f32 accumulate; "
                 f"prefill: fp16 MFMA operands, f32 accumulate; routing f32/f64 exact",
        "data": "synthetic (seeded N(0,0.02) experts in the config's encoding, F32 router N(0,1/sqrt(d)), x ~ N(0,1))",
        "config": {"workload": f"{desc}, T={args.tokens}",
                   "tokens": args.tokens, "d": spec.d, "d_ff": spec.d_ff, "E": spec.E, "k": spec.k,
                   "mode": (f"hipgraph ({GRAPH_CALLS} calls per graph)" if h["graph_us"] is not None and h["graph_us"] <= h["eager_us"] else "eager"),
                   "prefill_pack": packed},
        "roofline": {"kernel": (f"one-token slice kernel ({em.TYPE_NAMES[spec.wtype]}): router + routing, then per "
                                f"64-column slice of d_ff its gate/up rows, SwiGLU and down columns"
                                if h["path_bits"] & em.PATH_SLICES else
                                f"gate/up + SwiGLU expert kernel ({em.TYPE_NAMES[spec.wtype]})"
                                + (", router + routing fused in (one token)" if args.tokens == 1 else "")),
                     "bound": "hbm", "achieved": h["gate_up_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": h["gate_up_gbs"] / HBM_PEAK_GBS, "traffic": profiled_traffic(traffic_key, args.tokens),
                     "bytes_per_launch": algorithmic(spec, args.tokens, h["experts_hit"], h["path_bits"])[0],
                     "avg_launch_us": h["gate_up_us"]},
        "layer_hbm_frac": h["layer_hbm_frac"],
        "sweep": [results[T] for T in sweep_T],
    }
    if args.config == "c2" and not args.no_nested:
        # the other single-layer BASELINE configs (1, 3, 4) at their own token counts, nested so that the
        # default run records them too
        for name in ("c1", "c3", "c4"):
            try:
                line[name] = nested_config(em, name, max(5, args.steps // 2), args.warmup)
            except Exception as exc:
                line[name] = {"error": str(exc)}
    if args.config == "c2" and not args.no_c5:
        # BASELINE config 5 (the 32-layer Mixtral-architecture model, Q4_K experts) end to end, in the same
        # run: its own line's figures, nested here so the default run records them too
        try:
            line["c5"] = run_e2e(log_prefix="[bench c5]")
        except Exception as exc:
            line["c5"] = {"value": None, "error": str(exc)}
    if not args.no_cpu:
        try:
            line["cpu_baseline"] = cpu_baseline(hl, spec, sweep_T)
            for p in line["cpu_baseline"]["prefill"]:
                for r in line["sweep"]:
                    if r["T"] == p["T"]:
                        r["cpu_tokens_per_s"] = p["value"]
        except Exception as exc:
            line["cpu_baseline"] = {"value": None, "error": str(exc)}
    print(json.dumps(line), flush=True)


def run_e2e(prompt_len=512, n_new=256, log_prefix="[bench]"):
    """a random-init Mixtral-8x7B-architecture model (32 layers, Q4_K experts) through
    ember_moe/mixtral.py: seeded uniform-random prompt ids, prefill, then greedy decode steps at batch 1
    replayed from one captured HIP graph. Returns the figures; value = (prompt + generated tokens) / s."""
    import torch
    from ember_moe import mixtral

    spec = mixtral.MixtralSpec()
    model = mixtral.Mixtral(spec, max_ctx=prompt_len + n_new, log=lambda *a: log(log_prefix, *a))
    prompt = torch.from_numpy(np.random.default_rng(0).integers(0, spec.vocab, prompt_len)).cuda()
    model.generate(prompt[:16], 4)  # warm-up: kernels, the decode graph's code paths
    first, toks, t_pre, t_dec = model.generate(prompt, n_new)
    total = t_pre + t_dec
    # the same decode steps without the MoE FFN calls: the difference is the FFN's time per token
    _, _, _, t_dec_nomoe = model.generate(prompt, n_new, skip_moe=True)
    out = {
        "metric": "end-to-end tokens/s (c5)",
        "value": (prompt_len + n_new) / total,
        "unit": "tokens/s",
        "config": {"workload": f"config 5: Mixtral-8x7B architecture, {spec.n_layers} layers, prefill {prompt_len} + "
                               f"{n_new} greedy decode steps, batch 1", "expert_gb": model.expert_bytes / 1e9,
                   "decode": "one HIP graph per step"},
        "dtype": "q4_k experts through ember_moe_ffn; attention, norms, head bf16/fp32 PyTorch",
        "data": "synthetic (random-init weights, seeded uniform-random prompt ids)",
        "prefill_tokens_per_s": prompt_len / t_pre,
        "decode_tokens_per_s": n_new / t_dec,
        "prefill_s": t_pre,
        "decode_s": t_dec,
        "decode_moe_ms_per_token": (t_dec - t_dec_nomoe) / n_new * 1e3,
        "decode_moe_us_per_layer": (t_dec - t_dec_nomoe) / n_new / spec.n_layers * 1e6,
        "decode_moe_share": (t_dec - t_dec_nomoe) / t_dec,
        "first_tokens": [int(first[0])] + [int(t) for t in toks[:8].cpu()],
    }
    del model
    torch.cuda.empty_cache()
    return out


def bench_e2e(args):
    """bench.py --config c5: the end-to-end run alone, as its own JSON line."""
    r = run_e2e(n_new=args.decode_steps)
    line = {"metric": r["metric"], "value": r["value"], "unit": r["unit"], "n_gpus": 1, "steps": 1, "warmup": 1,
            "ms_per_step": (r["prefill_s"] + r["decode_s"]) * 1e3, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": r["dtype"], "data": r["data"], "config": r["config"]}
    line.update({k: v for k, v in r.items() if k not in line and k != "metric"})
    print(json.dumps(line), flush=True)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip() + f" ({os.cpu_count()} logical cpus visible)"
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
