"""MoE-FFN layer benchmark on one MI355X.

A step is one call of the whole MoE FFN layer (router, routed experts,
shared expert) over one batch of synthetic tokens, through the C ABI
(dsmoe_forward).  The default workload is BASELINE.json's quoted config:
the full-shape layer (d=7168, 256 experts in 8 groups, top-8, I=2048, Q8_0
shared expert) at decode B=1.  Steps rotate over `--layers` distinct weight
copies and 16 distinct token batches so consecutive steps do not hit the
same weights in the 256 MB last-level cache, as a stack of layers would not.

Prints ONE JSON line (rank 0) with `roofline` (dominant kernel, HIP events
on the launch stream) and `cpu_baseline` (the CPU oracle on host cores).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "deepseek-rs_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense f16 MFMA, MI355X
MFMA_I8_PEAK_TOPS = 5000.0  # dense int8 MFMA, MI355X
# the matrix-core type each grouped kernel's main product runs on (dn_grouped
# multiplies exact int8 weight and activation codes; the others f16)
STAGE_MFMA = {"gu_grouped": ("f16", MFMA_PEAK_TFLOPS), "dn_grouped": ("int8", MFMA_I8_PEAK_TOPS),
              "shared_up": ("f16", MFMA_PEAK_TFLOPS), "shared_dn": ("f16", MFMA_PEAK_TFLOPS)}


def prefill_flops(cfg, T):
    """Algorithmic MFMA flops of one grouped-path layer call, per kernel:
    2 flops per multiply-add of the routed and shared expert products."""
    d, I, Is, k = cfg.d_model, cfg.d_ff, cfg.d_ff_shared, cfg.top_k
    P = T * k
    return {"gu_grouped": P * 4 * I * d, "dn_grouped": P * 2 * d * I,
            "shared_up": T * 4 * Is * d if cfg.shared_fmt == 0 else 0,
            "shared_dn": T * 2 * d * Is if cfg.shared_fmt == 0 else 0}


PREFILL_KERNEL = {"gu_grouped": "dsmoe_gu_grouped", "dn_grouped": "dsmoe_dn_grouped",
                  "shared_up": "dsmoe_q80_gemm_swiglu_j7", "shared_dn": "dsmoe_q80_gemm_j2"}


def prefill_bench(case, steps, warmup, dev):
    """The 2048-token prefill config: whole-layer tokens/s and, per grouped
    kernel, achieved MFMA TFLOP/s from events around each launch."""
    import torch
    import dsmoe
    from dsmoe import configs as C
    cfg, T = case.cfg, case.T
    # the shared expert unpacked once per weight load, as an engine would
    w = C.make_weights(case, layer=0, device=dev).unpack_shared(cfg)
    xs = [C.make_x(case, T=T, step=s, device=dev) for s in range(2)]
    layer = dsmoe.MoeLayer(cfg, T)
    d, k = cfg.d_model, cfg.top_k
    so, ro = torch.empty(T, d, device=dev), torch.empty(T, d, device=dev)
    sel = torch.empty(T, k, dtype=torch.int32, device=dev)
    wt = torch.empty(T, k, device=dev)
    step = lambda i: layer.forward(w, xs[i % 2], so, ro, sel, wt)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        step(i)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    layer.set_profiling(True)
    layer.profile_read(reset=True)
    for i in range(steps):
        step(i)
    stages = layer.profile_read(reset=True)
    layer.set_profiling(False)
    fl = prefill_flops(cfg, T)
    rows = {}
    for name, (tot, n) in stages.items():
        avg = tot / max(n, 1)
        row = {"avg_us": round(avg * 1e3, 1)}
        if fl.get(name):
            row["flops"] = int(fl[name])
            row["TFLOPs"] = round(fl[name] / (avg * 1e-3) / 1e12, 1)
            typ, peak = STAGE_MFMA[name]
            row["mfma_type"], row["frac_of_type_peak"] = typ, round(row["TFLOPs"] / peak, 4)
        rows[name] = row
    dom = max((n for n in rows if "flops" in rows[n]), key=lambda n: rows[n]["avg_us"])
    tot_fl = sum(fl.values())
    import numpy as np
    counts = np.bincount(sel.cpu().numpy().reshape(-1), minlength=cfg.n_expert)
    layer.close()
    del w, xs
    where = ("added to the router logits (router column 0 = f16(-s ln rank), x[:, 0] = 1)" if case.zipf_logit
             else "added to the selection bias (score space, after sqrt(softplus))")
    return {
        "workload": f"{case.name}: same layer, T={T} tokens, Zipf({case.zipf}) expert popularity prior {where}",
        "experts_used": int(np.count_nonzero(counts)),
        "top10_share": round(float(np.sort(counts)[::-1][:10].sum() / counts.sum()), 4),
        "tokens_per_s": round(T / (ms * 1e-3), 1), "ms_per_step": round(ms, 4), "steps": steps,
        "mfma_flops_per_step": int(tot_fl), "achieved_TFLOPs": round(tot_fl / (ms * 1e-3) / 1e12, 1),
        "frac_of_mfma_peak": round(tot_fl / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
        "mfma_dtype": "f16 (exact small-integer operands, f32 accumulation) for gate/up and the shared expert; "
                      "int8 (exact, i32 accumulation) for the routed down projection; frac_of_mfma_peak and each "
                      "stage's TFLOPs count 2 flops per multiply-add against the f16 peak, frac_of_type_peak "
                      "against the peak of the type the stage runs on",
        "roofline": {"bound": "mfma", "kernel": PREFILL_KERNEL[dom], "achieved": rows[dom]["TFLOPs"],
                     "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(rows[dom]["TFLOPs"] / MFMA_PEAK_TFLOPS, 4),
                     "algorithmic_flops": rows[dom]["flops"],
                     "traffic": measured_traffic(PREFILL_KERNEL[dom], case.name, "grouped")},
        "stages": rows,
        "stage_mode": "solo: stage profiling runs every stage on the launch stream (no side stream), so each "
                      "kernel's time is its own; ms_per_step is the layer as run, shared expert forked",
    }


def stage_bytes(cfg, T, n_distinct):
    """Algorithmic HBM bytes per launch of each decode stage (T <= 8): weights
    streamed once, plus activations in and out.  "prep" = router logits +
    quantized x; "up" = routing, routed + shared gate/up/SwiGLU and the
    quantized mid rows; "dn" = routed down + slot sum + shared down."""
    d, I, E, Is, k = cfg.d_model, cfg.d_ff, cfg.n_expert, cfg.d_ff_shared, cfg.top_k
    iq2_row = (d // 256) * 66
    q2k_row = (I // 256) * 84
    if cfg.shared_fmt == 0:
        sh_up, sh_dn = 2 * Is * (d // 32) * 34, d * (Is // 32) * 34
    elif cfg.shared_fmt == 1:
        sh_up, sh_dn = 2 * Is * iq2_row, d * (Is // 256) * 84
    else:
        sh_up = sh_dn = 0
    return {
        "prep": E * d * 2 + T * d * 4 + T * E * 4 + T * (d // 256) * 292 + T * d * 9 // 8,
        "up": n_distinct * 2 * I * iq2_row + sh_up + T * k * I * 4 + T * k * (I // 256) * 292 + T * Is * 4
              + T * Is * 9 // 8,
        "dn": n_distinct * d * q2k_row + sh_dn + T * k * (I // 256) * 292 + T * Is * 9 // 8 + 2 * T * d * 4,
    }


STAGE_KERNEL = {"prep": "dsmoe_prep", "select": "dsmoe_router_select", "up": "dsmoe_up_rows", "midq": "dsmoe_midq",
                "dn": "dsmoe_dn_rows"}


def code_object_hash(kernel):
    """First 16 hex digits of the SHA-256 of the code object holding `kernel`
    (deepseek-rs_amd/profile_summary.py, which stamps the same hash on every
    profile line)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("dsmoe_profile_summary",
                                                  os.path.join(ROOT, "deepseek-rs_amd", "profile_summary.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.code_object_hash(kernel)


def measured_traffic(kernel, config, path, profiles=None):
    """HBM bytes per dispatch of `kernel` from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summaries (profiles/moe_<decode|prefill>_<config>_traffic.txt,
    counters scaled by a copy kernel of known size).  A summary line names
    the code object it was measured on (code_object=<hash>); a line for
    another build is stale and gives None, as does a kernel never measured."""
    profiles = profiles or os.path.join(ROOT, "profiles")
    want = code_object_hash(kernel)
    for kind in ("decode", "prefill"):
        f = os.path.join(profiles, f"moe_{kind}_{config}_traffic.txt")
        if not os.path.exists(f):
            continue
        for line in open(f):
            if not line.startswith("traffic "):
                continue
            kv = dict(t.split("=", 1) for t in line.split()[1:])
            if kv.get("kernel") == kernel and kv.get("config") == config and kv.get("path") == path:
                return int(kv["bytes"]) if want and kv.get("code_object") == want else None
    return None


def layer_bytes(cfg, n_distinct):
    return n_distinct * cfg.bytes_per_expert() + cfg.bytes_shared() + cfg.bytes_router()


def box_peaks(dev):
    """What this GPU sustains with no algorithm around it (dsmoe_probe):
    dense f16 MFMA TFLOP/s and HBM read GB/s, reported next to the
    published peaks the roofline fractions use."""
    import torch
    import dsmoe
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.zeros(8 * cus, device=dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    iters = 4096
    dsmoe.probe(0, None, 0, 64, sink)
    torch.cuda.synchronize()
    a.record()
    dsmoe.probe(0, None, 0, iters, sink)
    b.record()
    torch.cuda.synchronize()
    waves = 2 * cus * 4
    mfma = waves * iters * 8 * 32768 / (a.elapsed_time(b) * 1e-3) / 1e12
    buf = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    dsmoe.probe(1, buf, buf.numel(), 0, sink)
    torch.cuda.synchronize()
    a.record()
    for _ in range(5):
        dsmoe.probe(1, buf, buf.numel(), 0, sink)
    b.record()
    torch.cuda.synchronize()
    hbm = 5 * buf.numel() / (a.elapsed_time(b) * 1e-3) / 1e9
    del buf
    return {"mfma_f16_dense_TFLOPs": round(mfma, 1), "hbm_read_GBps": round(hbm, 1), "cus": cus,
            "note": "dsmoe_probe: 8 independent v_mfma_f32_32x32x16_f16 chains per wave, 2 waves per SIMD; "
                    "one 2 GiB read with 16-byte nontemporal loads"}


def host_info():
    model = "?"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


def config_bench(case, ws, steps, warmup, dev):
    """Tokens/s of one more config on the same library path, with the
    layer's algorithmic HBM bytes (router, the distinct experts' weights,
    shared expert) and, for the grouped path, its MFMA flops.  `ws` is a list
    of weight sets the steps rotate over (decode-sized configs get enough
    copies that a step's weights come from HBM, not the last-level cache)."""
    import numpy as np
    import torch
    import dsmoe
    from dsmoe import configs as C
    cfg, T = case.cfg, case.T
    xs = [C.make_x(case, T=T, step=s, device=dev) for s in range(4)]
    layer = dsmoe.MoeLayer(cfg, T)
    d, k = cfg.d_model, cfg.top_k
    so, ro = torch.empty(T, d, device=dev), torch.empty(T, d, device=dev)
    sel = torch.empty(T, k, dtype=torch.int32, device=dev)
    wt = torch.empty(T, k, device=dev)
    step = lambda i: layer.forward(ws[i % len(ws)], xs[i % len(xs)], so, ro, sel, wt)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        step(i)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    distinct = []
    for i in range(len(xs)):
        step(i)
        distinct.append(len(np.unique(sel.cpu().numpy())))
    nd = float(np.mean(distinct))
    lb = layer_bytes(cfg, nd)
    row = {"T": T, "weights_rotated": len(ws), "tokens_per_s": round(T / (ms * 1e-3), 1), "ms_per_step": round(ms, 4),
           "distinct_experts": nd, "algorithmic_bytes": int(lb),
           "hbm_frac": round(lb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if T > 8:
        fl = sum(prefill_flops(cfg, T).values())
        row["mfma_flops"] = int(fl)
        row["mfma_frac"] = round(fl / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4)
    layer.close()
    return row


def host_weights(w):
    import numpy as np
    f = lambda t: None if t is None else t.cpu().numpy().reshape(-1).copy()
    return {"router": w.router_f16.cpu().numpy().view(np.uint16).reshape(-1).copy(), "bias": f(w.bias),
            "gate": f(w.gate), "up": f(w.up), "down": f(w.down), "sh_gate": f(w.sh_gate), "sh_up": f(w.sh_up),
            "sh_down": f(w.sh_down)}


def cpu_baseline(case, hw, xs, seconds, cores, tokens=None):
    """The CPU oracle (a restatement of the reference arithmetic) on a
    bounded sample of the same workload: repeated layer calls over the first
    `tokens` tokens of each batch (all of them by default), for about
    `seconds` and at least one call."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_ref as O
    T = xs[0].shape[0] if tokens is None else min(tokens, xs[0].shape[0])
    xh = [x[:T].cpu().numpy().copy() for x in xs]
    n = 0
    t0 = time.perf_counter()
    while True:
        O.moe_forward(case.cfg, hw, xh[n % len(xh)], T, cores)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 2000:
            break
    return {"value": n * T / el, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} layer call{'s' if n > 1 else ''} x {T} token(s) of config {case.name} in {el:.1f} s "
                      f"(oracle/dsmoe_oracle.c, {cores} thread{'s' if cores > 1 else ''}, layer-0 weights)"}


# Tokens per CPU oracle call (every core, 1 thread): c1, c3 and c4 in full at
# every core; c5 (2048 tokens, ~1 min per call at 16 threads) on its first
# 64; 1-thread runs on the first 4 tokens of the batch configs.
CPU_TOKENS = {"c1": (None, None), "c2": (None, None), "c3": (None, 4), "c4": (None, 4), "c4tie": (None, 4), "c5": (64, 4),
              "c5logit": (64, 4)}


def cpu_pair(case, hw, xs, seconds, tokens_n, tokens_1):
    """The CPU oracle at every host core (the baseline) and at 1 thread, each
    for about `seconds` on a bounded sample of the config's tokens."""
    n = os.cpu_count() or 1
    multi = cpu_baseline(case, hw, xs, seconds, n, tokens_n)
    one = cpu_baseline(case, hw, xs, seconds, 1, tokens_1)
    return {"tokens_per_s": round(multi["value"], 3), "threads": n, "sample": multi["sample"],
            "tokens_per_s_1_thread": round(one["value"], 3), "sample_1_thread": one["sample"]}


def cpu_main(case, hw, xs, seconds):
    """cpu_baseline of the bench line: the oracle at every host core (value,
    cores) with the 1-thread figure beside it."""
    nproc = os.cpu_count() or 1
    tn, t1 = CPU_TOKENS.get(case.name, (None, None))
    cpu = cpu_baseline(case, hw, xs, seconds, nproc, tn)
    one = cpu_baseline(case, hw, xs, seconds / 2, 1, t1)
    cpu["host"] = host_info()
    cpu["value_1_thread"] = round(one["value"], 3)
    cpu["sample_1_thread"] = one["sample"]
    return cpu


def case_host_weights(case, hw_full, dev):
    """Host copies of a config's weights for the CPU oracle.  Configs that
    share C2's expert tensors (same shape and seed) reuse `hw_full` and take
    only their own router and bias."""
    import numpy as np
    import torch
    import dsmoe
    from dsmoe import configs as C
    if hw_full is not None and case.cfg == C.C2_CFG and case.seed == C.CASES["c2"].seed:
        E, d = case.cfg.n_expert, case.cfg.d_model
        seed = case.seed
        if case.router_tie:  # every expert's router row the same: routing decided by the bias and ties
            row = dsmoe.synth(dsmoe.FMT_F16, seed, C.TID_ROUTER, 1, 1, d, sigma=0.02, device="cpu")
            router = row.reshape(1, d).expand(E, d).contiguous()
        else:
            router = dsmoe.synth(dsmoe.FMT_F16, seed, C.TID_ROUTER, 1, E, d, sigma=0.02, device="cpu")
        bias = dsmoe.synth(dsmoe.FMT_F32, seed, C.TID_BIAS, 1, 1, E, sigma=0.01, device="cpu").reshape(E).clone()
        if case.zipf > 0 and case.zipf_logit:
            prior = torch.from_numpy(C.zipf_bias(E, case.zipf, seed)).to(torch.float16)
            router = router.clone()
            router[:, 0] = prior.view(torch.int16)
        elif case.zipf > 0:
            bias += torch.from_numpy(C.zipf_bias(E, case.zipf, seed))
        hw = dict(hw_full)
        hw["router"] = router.numpy().view(np.uint16).reshape(-1).copy()
        hw["bias"] = bias.numpy().copy()
        return hw
    w = C.make_weights(case, layer=0, device=dev)
    hw = host_weights(w)
    del w
    return hw


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--prefill-config", default="c5,c5logit",
                    help="configs of the prefill measurement added to the line, comma-separated ('none' to skip); "
                         "c5 is reported under prefill, the others under prefill_variants")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--other-configs", default="c1,c3,c4,c4tie",
                    help="configs also timed on the same path, reported under other_configs ('none' to skip)")
    ap.add_argument("--no-peaks", action="store_true", help="skip the on-box MFMA / HBM peak probes")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay timing of the decode step")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every box in this build has one MI355X and the MoE path is "
              f"single-GPU (see DESIGN.md, 'How it would shard'); got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import dsmoe
    from dsmoe import configs as C

    dev = torch.device("cuda:0")
    dsmoe.init()
    case = C.CASES[args.config]
    cfg, T = case.cfg, case.T
    L = max(1, args.layers)
    print(f"[bench] config={case.name} T={T} layers={L}: generating weights", file=sys.stderr, flush=True)
    layers = [C.make_weights(case, layer=i, device=dev) for i in range(L)]
    if T > 8:  # batches: the shared expert unpacked once per weight load, as an engine would
        layers = [w.unpack_shared(cfg) for w in layers]
    xs = [C.make_x(case, T=T, step=s, device=dev) for s in range(16)]
    layer = dsmoe.MoeLayer(cfg, T)
    path = "staged"
    d, k = cfg.d_model, cfg.top_k
    so = torch.empty(T, d, device=dev)
    ro = torch.empty(T, d, device=dev)
    sel = torch.empty(T, k, dtype=torch.int32, device=dev)
    wt = torch.empty(T, k, device=dev)
    torch.cuda.synchronize()

    def step(i):
        layer.forward(layers[i % L], xs[i % len(xs)], so, ro, sel, wt)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    print("[bench] timing", file=sys.stderr, flush=True)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        step(i)
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps

    # the same steps replayed from HIP graphs.  A graph holds kGraphSteps
    # consecutive layer calls (rotating weights and activations, as a
    # captured decode step over a stack of layers would): each graph launch
    # costs the GPU a fixed idle gap (about 8 us between the end of one
    # replay and the start of the next, measured with a kernel trace; no gap
    # appears between the kernel nodes inside a replay), which one call per
    # graph would pay per layer.
    graph_ms = None
    kGraphSteps = 64
    if T <= 8 and not args.no_graph:
        cs = torch.cuda.Stream()
        cs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cs):
            step(0)
        torch.cuda.current_stream().wait_stream(cs)
        graphs = []
        for gi in range(2):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for i in range(kGraphSteps):
                    step(gi * kGraphSteps + i)
            graphs.append(gr)
        reps = max(1, args.steps // kGraphSteps)
        for i in range(2):
            graphs[i % 2].replay()
        torch.cuda.synchronize()
        start.record()
        for i in range(reps):
            graphs[i % 2].replay()
        stop.record()
        torch.cuda.synchronize()
        graph_ms = start.elapsed_time(stop) / (reps * kGraphSteps)
        del graphs

    # per-stage timing pass (events around each stage on the launch stream)
    nprof = min(args.steps, 100)
    distinct = []
    layer.set_profiling(True)
    layer.profile_read(reset=True)
    for i in range(nprof):
        step(i)
        distinct.append(len(np.unique(sel.cpu().numpy())))
    stages = layer.profile_read(reset=True)
    layer.set_profiling(False)
    nd = float(np.mean(distinct))
    sb = stage_bytes(cfg, T, nd)
    stage_rows = {}
    for name, (tot, n) in stages.items():
        avg = tot / max(n, 1)
        row = {"avg_us": round(avg * 1e3, 2)}
        if name in sb:
            row["algorithmic_bytes"] = int(sb[name])
            row["GBps"] = round(sb[name] / (avg * 1e-3) / 1e9, 1)
        stage_rows[name] = row
    dom = max((n for n in stage_rows if "algorithmic_bytes" in stage_rows[n]),
              key=lambda n: stage_rows[n]["avg_us"])
    ach = stage_rows[dom]["GBps"]
    lb = layer_bytes(cfg, nd)
    layer_gbs = lb / (ms * 1e-3) / 1e9

    if args.copy_calibration:
        src = torch.ones(64 << 20, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    prefill = {}
    if args.prefill_config != "none":
        for name in [n for n in args.prefill_config.split(",") if n and n != args.config]:
            print(f"[bench] prefill {name}", file=sys.stderr, flush=True)
            prefill[name] = prefill_bench(C.CASES[name], args.prefill_steps, 2, dev)

    others = {}
    if args.other_configs != "none":
        for name in [n for n in args.other_configs.split(",") if n and n != args.config]:
            oc = C.CASES[name]
            print(f"[bench] config {name}", file=sys.stderr, flush=True)
            # the decode config's weights serve configs of the same layer and router
            same = (oc.cfg == cfg and oc.seed == case.seed and oc.d_ff_real == case.d_ff_real and
                    oc.router_tie == case.router_tie and oc.zipf == case.zipf and oc.zipf_logit == case.zipf_logit)
            if same:
                ow = layers if oc.T <= 8 else layers[:1]
            else:  # decode-sized configs rotate over enough copies to exceed the 256 MB last-level cache
                nl = max(1, -(-(512 << 20) // layer_bytes(oc.cfg, oc.cfg.n_expert))) if oc.T <= 8 else 1
                ow = [C.make_weights(oc, layer=i, device=dev) for i in range(nl)]
                if oc.T > 8:
                    ow = [w.unpack_shared(oc.cfg) for w in ow]
            others[name] = config_bench(oc, ow, 50 if oc.T <= 8 else 20, 5, dev)
            del ow

    peaks = None
    if not args.no_peaks:
        print("[bench] peak probes", file=sys.stderr, flush=True)
        peaks = box_peaks(dev)

    cpu = None
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        hw = host_weights(layers[0])
        cpu = cpu_main(case, hw, xs, args.cpu_seconds)
        # the same oracle beside every other config's GPU figure
        for name, row in list(others.items()) + list(prefill.items()):
            oc = C.CASES[name]
            print(f"[bench] cpu baseline {name}", file=sys.stderr, flush=True)
            ohw = case_host_weights(oc, hw, dev)
            oxs = [C.make_x(oc, T=oc.T, step=s, device="cpu") for s in range(2)]
            tn, t1 = CPU_TOKENS.get(name, (None, 4))
            row["cpu"] = cpu_pair(oc, ohw, oxs, args.cpu_seconds / 4, tn, t1)
            row["gpu_over_cpu"] = round(row["tokens_per_s"] / row["cpu"]["tokens_per_s"], 1)
            del ohw

    out = {
        "metric": "MoE-layer tokens/s & % of HBM/MFMA roofline, decode B=1 and prefill 2048",
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic",
        "config": {"workload": f"{case.name}: full MoE FFN layer, d={d}, E={cfg.n_expert} "
                               f"({cfg.n_group} groups, top-{cfg.topk_group}), top-{k}, I={cfg.d_ff}, "
                               f"shared={'Q8_0' if cfg.shared_fmt == 0 else 'IQ2_XXS/Q2_K'} I_s={cfg.d_ff_shared}, "
                               f"T={T}", "global_batch": T, "weights_rotated": L, "distinct_experts": nd},
        "roofline": {"bound": "hbm", "kernel": STAGE_KERNEL.get(dom, dom), "achieved": ach, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": stage_rows[dom]["algorithmic_bytes"],
                     "traffic": measured_traffic(STAGE_KERNEL.get(dom, dom), case.name, path)},
        "layer_roofline": {"algorithmic_bytes": int(lb), "achieved": round(layer_gbs, 1), "unit": "GB/s",
                           "frac": round(layer_gbs / HBM_PEAK_GBS, 4)},
        "stages": stage_rows,
        "graph_replay": None if graph_ms is None else {
            "ms_per_step": round(graph_ms, 5), "tokens_per_s": round(T / (graph_ms * 1e-3), 1),
            "steps_per_graph": kGraphSteps,
            "note": f"the same layer calls captured {kGraphSteps} to a HIP graph (rotating weight sets and "
                    f"activations) and replayed; one graph launch costs an ~8 us idle gap on the GPU, so a graph "
                    f"per layer call would be slower than eager launches"},
        "prefill": prefill.get("c5"),
        "prefill_variants": {n: v for n, v in prefill.items() if n != "c5"},
        "other_configs": others,
        "box_peaks": peaks,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
