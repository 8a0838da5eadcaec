"""Benchmark of the fused low-rank LM-head argmax (DeLS draft-token selection) on one MI355X.

One step = one draft step of the hot path on one batch: the rank projection
rank = bf16(h . A^T) and the fused combine + vocabulary argmax over B [V, r],
base logits [M, V] and the log-prior [V], with all inputs resident in HBM.
The default workload is the Qwen3-8B low-rank head at M=16 (d=4096, r=512,
V=151936, fp32 base logits, per-position alpha/beta); ``--also-m512`` adds the
batched M=512 shape (bf16 base and prior) as a second, informative record.

Timing: ``--sets`` input sets (> 256 MB in total, so B cannot stay resident in
the 256 MB MALL) are rotated step by step.  The K timed steps are one hipGraph
of K consecutive draft steps (kernels back to back, no host launch overhead),
bracketed by torch.cuda.synchronize() and HIP events on the launch stream.
With packed weights at M <= 16 a step is one launch of the decode kernel
(rank projection and fused argmax in one kernel), so the step graph times that
kernel directly; at M=512 the dominant kernel, the fused argmax, is timed by a
second graph of K argmax launches only (rank precomputed), the same way.  The
argmax-only graph is reported at M=16 too, as a secondary figure.

CPU baseline: the reference's eager CPU PyTorch step (F.linear, bf16 combine,
torch.argmax; restated in oracle/torch_eager.py) on the same inputs, median of
at least 20 calls on the host's CPU share, with its id agreement with the GPU.
``--cpu-configs`` times it at every configuration instead and prints a table.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import platform
import sys
import time

REPO_DIR = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO_DIR)

METRIC = "argmax rows/s + % HBM/MFMA roofline, Qwen3-8B low-rank LM head, M=16 & 512"
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
FP8_MFMA_PEAK_TFLOPS = 5000.0


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="qwen3_8b_m16", choices=["qwen3_8b_m16", "qwen3_4b_m16", "qwen3_8b_m512"])
    ap.add_argument("--sets", type=int, default=0, help="rotating input sets (0: enough for > 512 MB)")
    ap.add_argument("--also-m512", action=argparse.BooleanOptionalAction, default=True)
    ap.add_argument("--also-draft-step", action=argparse.BooleanOptionalAction, default=True,
                    help="add the whole draft block (target LM head + first argmax + DeLS rollout, one graph)")
    ap.add_argument("--also-fp8", action=argparse.BooleanOptionalAction, default=True,
                    help="add the fp8 variant (e4m3 A and B with per-channel scales) of the workload's shape")
    ap.add_argument("--also-batched-lm-head", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the target LM head at M=512 (library GEMM and the hand-written kernel)")
    ap.add_argument("--also-domino", action=argparse.BooleanOptionalAction, default=True,
                    help="add one Domino correction step (code/kernel/domino.py:58-173) at the draft block's batch")
    ap.add_argument("--cpu-baseline", action=argparse.BooleanOptionalAction, default=True)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-configs", action="store_true",
                    help="only time the reference's CPU torch step at every configuration (no GPU use); "
                         "one JSON line per configuration")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy a 512 MiB buffer 8 times (scale reference for HBM byte counters)")
    ap.add_argument("--layout", default="packed", choices=["packed", "rowmajor"],
                    help="weights in the MFMA-16 block layout (as the runner stores them) or row-major")
    ap.add_argument("--traffic-file", default=os.path.join(REPO_DIR, "profiles", "traffic.json"))
    ap.add_argument("--traffic-from", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV", "COPY_WRITE_CSV"),
                    help="turn rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE counter CSVs of a bench run and of a "
                         "--copy-calibration run into per-launch HBM bytes (written to --traffic-file); no GPU use")
    return ap.parse_args()


# The dominant kernel(s) of one step per workload, with packed weights.  At
# M <= 16 the whole step (rank projection + fused argmax) is one launch of the
# decode kernel; at M=512 the step runs the rank projection GEMM, then the tiled
# argmax (its cross-workgroup reduce folded in), which dominates.
ROOFLINE_KERNELS = {"qwen3_8b_m16": ("lowrank_decode_kernel",),
                    "qwen3_4b_m16": ("lowrank_decode_kernel",),
                    "qwen3_8b_m512": ("fused_argmax_tiled_kernel",)}
# With row-major weights the M=16 step is the rank projection and the GEMV argmax.
ROWMAJOR_M16_KERNELS = ("fused_argmax_gemv_kernel",)


def step_is_one_launch(workload, layout):
    return layout == "packed" and workload in ("qwen3_8b_m16", "qwen3_4b_m16")


def _counter_means(path):
    """Mean counter value (KiB per dispatch) per (kernel substring match, counter) from a rocprofv3 CSV."""
    import csv
    import statistics
    per = {}
    with open(path) as fh:
        for row in csv.DictReader(fh):
            per.setdefault((row["Kernel_Name"], row["Counter_Name"]), []).append(float(row["Counter_Value"]))
    return {k: (statistics.mean(v), len(v)) for k, v in per.items()}


def traffic_from(args):
    """HBM bytes per launch of the argmax kernels from FETCH_SIZE / WRITE_SIZE counters.

    Each counter is scaled by the ratio of the bytes a plain copy kernel moves
    (512 MiB read, 512 MiB written per dispatch) to what the same counter reads
    for that copy.  The bench run holds the M=16 (GEMV) and M=512 (tiled)
    launches; the two are told apart by kernel name.
    """
    fetch, write, cfetch, cwrite = (_counter_means(p) for p in args.traffic_from)
    copy_bytes = 512 * 2**20

    def copy_scale(means, counter):
        vals = [m for (k, c), (m, n) in means.items() if c == counter and "copy" in k.lower()]
        if not vals:
            raise SystemExit(f"no copy kernel with {counter} in the calibration CSV")
        return copy_bytes / (max(vals) * 1024.0)

    fs, ws = copy_scale(cfetch, "FETCH_SIZE"), copy_scale(cwrite, "WRITE_SIZE")

    def kib(means, counter, names):
        total = 0.0
        for name in names:
            vals = [(m, n) for (k, c), (m, n) in means.items() if c == counter and name in k]
            if not vals:
                return None
            total += max(vals, key=lambda t: t[1])[0]
        return total

    out = {"fetch_scale": fs, "write_scale": ws,
           "method": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (KiB per dispatch, mean over dispatches), "
                     "each scaled by copy_bytes / counter of a 512 MiB device copy"}
    # the default bench run covers these two workloads (the M=16 record and the M=512 one)
    for wl in ("qwen3_8b_m16", "qwen3_8b_m512"):
        names = ROOFLINE_KERNELS[wl]
        f, w = kib(fetch, "FETCH_SIZE", names), kib(write, "WRITE_SIZE", names)
        if f is None or w is None:
            continue
        out[wl] = {"kernels": list(names), "fetch_kib": f, "write_kib": w,
                   "hbm_bytes_per_launch": f * 1024.0 * fs + w * 1024.0 * ws}
    with open(args.traffic_file, "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out))


def workload_desc(name, x, layout):
    s = x.shape
    return {
        "workload": name,
        "M": s["M"], "d": s["d"], "r": s["r"], "V": s["V"],
        "base_dtype": str(x.base.dtype).replace("torch.", ""),
        "prior_dtype": str(x.prior.dtype).replace("torch.", ""),
        "alpha_beta": "per-position U[0,0.6], period 16" if name != "qwen3_4b_m16" else "scalar 0.3",
        "act": x.act,
        "weights_layout": "MFMA-16 blocks" if layout == "packed" else "row-major",
    }


def kernel_bytes(M, d, r, V, base_bytes, prior_bytes):
    """Algorithmic HBM bytes of the fused argmax kernel and of the whole step."""
    argmax = 2 * r * V + base_bytes * M * V + prior_bytes * V + 2 * M * r + 12 * M
    rank = 2 * r * d + 2 * M * d + 2 * M * r
    return argmax, rank


def make_sets(pkg, x_cpu, nsets, dev):
    """Set 0: the seeded CPU inputs; sets 1..: the same distributions drawn on the GPU."""
    import torch

    x0 = x_cpu.to(dev)
    sets = [x0]
    g = torch.Generator(device=dev)
    for i in range(1, nsets):
        g.manual_seed(1000 + i)
        s = x0.shape
        h = torch.randn(s["M"], s["d"], generator=g, device=dev).to(torch.bfloat16)
        A = (torch.randn(s["r"], s["d"], generator=g, device=dev) * 0.02).to(torch.bfloat16)
        B = (torch.randn(s["V"], s["r"], generator=g, device=dev) * 0.02).to(torch.bfloat16)
        base = (torch.randn(s["M"], s["V"], generator=g, device=dev) * 3).to(x0.base.dtype)
        prior = x0.prior[torch.randperm(s["V"], generator=g, device=dev)].contiguous()
        sets.append(pkg.synth.LowRankInputs(h, A, B, base, prior, x0.alpha, x0.beta, x0.act))
    return sets


def set_bytes(x):
    return sum(t.numel() * t.element_size() for t in (x.h, x.A, x.B, x.base, x.prior))


def replay_stats(ms_list):
    """Median, p10, p90 and min of per-replay times (ms)."""
    xs = sorted(ms_list)
    q = lambda p: xs[min(len(xs) - 1, max(0, round(p * (len(xs) - 1))))]  # noqa: E731
    return {"median": q(0.5), "p10": q(0.1), "p90": q(0.9), "min": xs[0], "replays": len(xs)}


def time_graph(torch, record, steps, dev, reps=11):
    """Capture `record(i)` for i < steps in one graph; the median of `reps` timed replays (ms),
    with the spread of the replays (``replay_stats``) as a second value."""
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        record(0)                        # sizes this stream's workspace outside the capture
        torch.cuda.synchronize(dev)
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                record(i)
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize(dev)
    graph.replay()                       # warm replay
    torch.cuda.synchronize(dev)
    times = []
    cur = torch.cuda.current_stream(dev)
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        e0.record(cur)
        graph.replay()
        e1.record(cur)
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1))
    st = replay_stats(times)
    return st["median"], graph, st


def per_step_us(st, steps):
    """``replay_stats`` of graph replays of ``steps`` launches, as µs per launch."""
    return {k: (v * 1e3 / steps if k != "replays" else v) for k, v in st.items()}


def bench_workload(pkg, name, args, dev, torch, base_dtype=None):
    """``base_dtype``: base logits of that dtype instead of the configuration's (same values, cast)."""
    nsets = args.sets
    x0 = pkg.synth.config_inputs(name)
    if base_dtype is not None:
        x0 = dataclasses.replace(x0, base=x0.base.to(base_dtype))
    per = set_bytes(x0)
    if nsets <= 0:
        nsets = max(3, -(-512 * 2**20 // per))
    sets = make_sets(pkg, x0, nsets, dev)
    s = x0.shape
    M, d, r, V = s["M"], s["d"], s["r"], s["V"]
    outs = [(torch.empty(M, dtype=torch.int64, device=dev), torch.empty(M, dtype=torch.float32, device=dev))
            for _ in range(nsets)]
    ranks = [torch.empty(M, r, dtype=torch.bfloat16, device=dev) for _ in range(nsets)]
    if args.layout == "packed":
        # as the runner stores them: both weights in the MFMA-16 block layout
        weights = [(pkg.pack_operand(x.A), pkg.pack_operand(x.B)) for x in sets]
    else:
        weights = [(x.A, x.B) for x in sets]

    def step(i):
        x = sets[i % nsets]
        o = outs[i % nsets]
        A, B = weights[i % nsets]
        pkg.lowrank_argmax(x.h, A, B, x.base, x.prior, x.alpha, x.beta, act=x.act, out_ids=o[0], out_score=o[1])

    def argmax_only(i):
        x = sets[i % nsets]
        o = outs[i % nsets]
        pkg.fused_argmax(ranks[i % nsets], weights[i % nsets][1], x.base, x.prior, x.alpha, x.beta, out_ids=o[0],
                         out_score=o[1])

    # eager warm-up (also sizes the shared workspace before capture); every set
    # runs at least once, so each graph replay below has an eager result to match
    for i in range(max(args.warmup, nsets)):
        step(i)
    torch.cuda.synchronize(dev)
    eager = [(o[0].clone(), o[1].clone()) for o in outs]
    ids_set0 = eager[0][0].cpu()          # set 0 holds the seeded CPU inputs
    for i in range(nsets):
        pkg.rank_proj(sets[i].h, weights[i][0], None, sets[i].act, out=ranks[i])
    torch.cuda.synchronize(dev)

    ms_total, g_step, st_step = time_graph(torch, step, args.steps, dev)
    # the graph replays must reproduce the eager results
    for i in range(nsets):
        if not (torch.equal(outs[i][0], eager[i][0]) and torch.equal(outs[i][1], eager[i][1])):
            raise RuntimeError(f"graph replay differs from eager results on set {i}")
    ms_kernel_total, g_arg, st_arg = time_graph(torch, argmax_only, args.steps, dev)
    del g_step, g_arg

    ms_step = ms_total / args.steps
    us_kernel = ms_kernel_total * 1e3 / args.steps
    base_b = x0.base.element_size()
    prior_b = x0.prior.element_size()
    arg_bytes, rank_bytes = kernel_bytes(M, d, r, V, base_b, prior_b)
    flops_step = 2.0 * M * r * (d + V)
    rec = {
        "M": M, "d": d, "r": r, "V": V,
        "rows_per_s": M / (ms_step * 1e-3),
        "us_per_step": ms_step * 1e3,
        "us_fused_argmax": us_kernel,
        "argmax_bytes": arg_bytes,
        "step_bytes": arg_bytes + rank_bytes,
        "argmax_GBs": arg_bytes / (us_kernel * 1e-6) / 1e9,
        "step_GBs": (arg_bytes + rank_bytes) / (ms_step * 1e-3) / 1e9,
        "step_TFLOPs": flops_step / (ms_step * 1e-3) / 1e12,
        "sets": nsets,
        "set_MB": per / 2**20,
        "ids_set0": ids_set0,
        "us_per_step_spread": per_step_us(st_step, args.steps),
        "us_fused_argmax_spread": per_step_us(st_arg, args.steps),
    }
    rec["hbm_frac_step"] = rec["step_GBs"] / HBM_PEAK_GBS
    rec["mfma_frac_step"] = rec["step_TFLOPs"] / BF16_MFMA_PEAK_TFLOPS
    rec["argmax_TFLOPs"] = 2.0 * M * r * V / (us_kernel * 1e-6) / 1e12
    rec["argmax_mfma_frac"] = rec["argmax_TFLOPs"] / BF16_MFMA_PEAK_TFLOPS
    rec["argmax_hbm_frac"] = rec["argmax_GBs"] / HBM_PEAK_GBS
    return rec, x0



def bench_domino(pkg, args, dev, torch):
    """One Domino correction step, argmax_v alpha * (SiLU(z + s) . fc2[v]) + base[v] (code/kernel/domino.py:
    58-173), for the draft block's 8 rows at E = 1024, V = 151936, bf16 base, no fc2 bias: fc2 (311 MB, more
    than the 256 MB last-level cache) streamed once per step."""
    M, E, V = 8, 1024, 151936
    g = torch.Generator(device=dev).manual_seed(5)
    z = torch.randn(M, E, generator=g, device=dev).to(torch.bfloat16)
    s = torch.randn(M, E, generator=g, device=dev).to(torch.bfloat16)
    fc2 = pkg.pack_operand((torch.randn(V, E, generator=g, device=dev) * 0.02).to(torch.bfloat16))
    base = (torch.randn(M, V, generator=g, device=dev) * 3).to(torch.bfloat16)
    ids = torch.empty(M, dtype=torch.int64, device=dev)
    score = torch.empty(M, dtype=torch.float32, device=dev)
    steps = max(20, min(args.steps, 200))
    ms, graph, st = time_graph(torch, lambda i: pkg.domino_argmax(z, s, fc2, base, 0.7, out_ids=ids,
                                                                  out_score=score), steps, dev)
    del graph
    us = ms * 1e3 / steps
    nbytes = 2 * V * E + 2 * M * V + 4 * M * E + 12 * M
    return {"workload": f"domino step: {M} rows, E {E}, V {V}, bf16 base, no bias", "kernel": "domino_argmax_kernel",
            "us_per_step": us, "rows_per_s": M / (us * 1e-6), "algorithmic_bytes": nbytes,
            "GBs": nbytes / (us * 1e-6) / 1e9, "hbm_frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "us_per_step_spread": per_step_us(st, steps)}


def fp8_id_agreement(pkg, x, w8, torch):
    """The fp8 step's ids against the bf16 path's on one input set, under the top-2 margin rule.

    Reference ids: the bf16 kernels on the unquantised weights (the GPU tests pin
    them to the oracle).  A row is "pinned" when the bf16 top-2 margin exceeds
    twice the row's bound on the fp8 error,
    ``max_v |alpha| (|eR|.(|B| + |eB|) + |rank|.|eB|)[v]`` (+1e-4 for fp32
    rounding), where ``eB`` is B's e4m3 rounding and ``eR`` the difference
    between the rank the fp8 MFMAs contract (the e4m3 A's rank, quantised per row
    as the kernels do) and the bf16 rank; all of it evaluated in fp64 on the
    device.  On pinned rows the ids must agree; elsewhere either pick is within
    rounding.
    """
    f64, f32 = torch.float64, torch.float32
    A8, B8 = w8
    ids8, _ = pkg.lowrank_argmax_fp8(x.h, A8, B8, x.base, x.prior, x.alpha, x.beta, act=x.act)
    ids_b, _ = pkg.lowrank_argmax(x.h, pkg.pack_operand(x.A), pkg.pack_operand(x.B), x.base, x.prior, x.alpha,
                                  x.beta, act=x.act)
    rank_b = pkg.rank_proj(x.h, x.A, None, x.act).to(f64)
    qA, sA = pkg.quantize_e4m3_rows(x.A)
    qB, sB = pkg.quantize_e4m3_rows(x.B)
    Ad = qA.view(torch.float8_e4m3fn).to(f64) * sA.to(f64)[:, None]
    Bd = qB.view(torch.float8_e4m3fn).to(f64) * sB.to(f64)[:, None]
    rank8 = (x.h.to(f64) @ Ad.t()).to(f32).to(torch.bfloat16)
    if x.act == "silu":
        rank8 = torch.nn.functional.silu(rank8.float()).to(torch.bfloat16)
    r8 = rank8.float()
    amax = r8.abs().amax(dim=1)
    nz = amax > 0
    inv = torch.where(nz, 448.0 / torch.where(nz, amax, torch.ones_like(amax)), torch.ones_like(amax))
    scl = torch.where(nz, amax / 448.0, torch.ones_like(amax))
    used = (r8 * inv[:, None]).to(torch.float8_e4m3fn).to(f64) * scl.to(f64)[:, None]
    Bf = x.B.to(f64)
    eB = (Bd - Bf).abs()
    eR = (used - rank_b).abs()
    alpha, beta = x.alpha.to(f64), x.beta.to(f64)
    E = alpha.abs()[:, None] * (eR @ (Bf.abs() + eB).t() + rank_b.abs() @ eB.t())
    Emax = E.amax(dim=1) + 1e-4
    del E
    sc = (rank_b @ Bf.t()) * alpha[:, None] + x.base.to(f64)
    sc = torch.where((beta != 0)[:, None], sc - beta[:, None] * x.prior.to(f64)[None, :], sc)
    top2 = torch.topk(sc, 2, dim=1).values
    del sc
    pinned = (top2[:, 0] - top2[:, 1]) > 2 * Emax
    match = ids8 == ids_b
    npin = int(pinned.sum())
    return {"rows": int(match.numel()), "match": float(match.float().mean()), "pinned_rows": npin,
            "pinned_match": float(match[pinned].float().mean()) if npin else None,
            "median_bound": float(Emax.median()),
            "reference": "bf16 kernels on the unquantised weights (seeded input set)"}


def bench_fp8(pkg, name, args, dev, torch):
    """The fp8 variant of a workload: e4m3 A and B (per-channel fp32 scales), same h/base/prior/alpha/beta.

    Algorithmic bytes per step: r*V (B) + r*d (A) + 2*M*d (h) + s_base*M*V +
    s_prior*V + 4*(V + r) (scales) + 12*M (outputs)."""
    x0 = pkg.synth.config_inputs(name)
    nsets = max(4, -(-512 * 2**20 // (set_bytes(x0) // 2)))
    sets = make_sets(pkg, x0, nsets, dev)
    s = x0.shape
    M, d, r, V = s["M"], s["d"], s["r"], s["V"]
    weights = [(pkg.quantize_pack_fp8(x.A, "k32"), pkg.quantize_pack_fp8(x.B, "k128")) for x in sets]
    ranks = [pkg.rank_proj(x.h, x.A, None, x.act) for x in sets]   # for the argmax-only timing
    agreement = fp8_id_agreement(pkg, sets[0], weights[0], torch)   # set 0: the seeded inputs
    for x in sets:   # the bf16 weights are not read by the fp8 step
        x.A = x.B = None
    torch.cuda.empty_cache()
    outs = [(torch.empty(M, dtype=torch.int64, device=dev), torch.empty(M, dtype=torch.float32, device=dev))
            for _ in range(nsets)]

    def step(i):
        x = sets[i % nsets]
        o = outs[i % nsets]
        A8, B8 = weights[i % nsets]
        pkg.lowrank_argmax_fp8(x.h, A8, B8, x.base, x.prior, x.alpha, x.beta, act=x.act, out_ids=o[0],
                               out_score=o[1])

    for i in range(max(args.warmup, nsets)):   # every set at least once before the capture
        step(i)
    torch.cuda.synchronize(dev)
    eager = [(o[0].clone(), o[1].clone()) for o in outs]
    steps = min(args.steps, 200)
    ms_total, g, st_step = time_graph(torch, step, steps, dev)
    del g
    for i in range(nsets):
        if not (torch.equal(outs[i][0], eager[i][0]) and torch.equal(outs[i][1], eager[i][1])):
            raise RuntimeError(f"fp8 graph replay differs from eager results on set {i}")
    us = ms_total * 1e3 / steps

    def argmax_only(i):
        x = sets[i % nsets]
        o = outs[i % nsets]
        pkg.fused_argmax_fp8(ranks[i % nsets], weights[i % nsets][1], x.base, x.prior, x.alpha, x.beta,
                             out_ids=o[0], out_score=o[1])

    argmax_only(0)
    torch.cuda.synchronize(dev)
    ms_arg, g, st_arg = time_graph(torch, argmax_only, steps, dev)
    del g
    us_arg = ms_arg * 1e3 / steps
    sb = x0.base.element_size()
    sp = x0.prior.element_size()
    nbytes = r * V + r * d + 2 * M * d + sb * M * V + sp * V + 4 * (V + r) + 12 * M
    arg_bytes = nbytes - r * d - 2 * M * d - 4 * r + 2 * M * r
    flops, arg_flops = 2 * M * r * (d + V), 2 * M * r * V
    tiled = M >= 64
    return {"workload": name, "M": M, "d": d, "r": r, "V": V, "weights": "e4m3 (A K32, B K128 blocks)",
            "kernel": "lowrank_decode8_kernel" if M <= 16 else
            ("rank_gemm_tiled_kernel (e4m3 A) + rank_splitk_epilogue_kernel (quantising)"
             " + fused_argmax_tiled8_kernel"
             if tiled else "skinny_gemm_kernel (e4m3 A) + fused_argmax_gemv8_kernel"),
            "rows_per_s": M / (us * 1e-6), "us_per_step": us, "algorithmic_bytes": nbytes,
            "GBs": nbytes / (us * 1e-6) / 1e9, "hbm_frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "mfma_frac": flops / (us * 1e-6) / 1e12 / FP8_MFMA_PEAK_TFLOPS,
            "sets": nsets,
            "us_per_step_spread": per_step_us(st_step, steps),
            "id_match_vs_bf16": agreement,
            "fused_argmax_only": {"kernel": "quantize_rank_e4m3_kernel + fused_argmax_tiled8_kernel"
                                            if tiled else "fused_argmax_gemv8_kernel",
                                  "us_per_launch": us_arg, "us_per_launch_spread": per_step_us(st_arg, steps),
                                  "algorithmic_bytes": arg_bytes,
                                  "hbm_frac": arg_bytes / (us_arg * 1e-6) / 1e9 / HBM_PEAK_GBS,
                                  "mfma_frac": arg_flops / (us_arg * 1e-6) / 1e12 / FP8_MFMA_PEAK_TFLOPS}}



def bench_draft_step(pkg, args, dev, torch):
    """One whole draft block as one graph: batch 8, block 16 unshifted (k_draft 15: one
    plain argmax + 14 DeLS steps), target LM head W [151936, 4096] bf16 ~ N(0, 0.02),
    local head hidden 1024 (embeddings 1024, rank 256, silu), per-position alpha/beta
    U[0, 0.6], the Zipf log-prior; hidden states ~ N(0, 1).

    The block as DeLSDraftStep builds it by default: the hand-written LM head
    (lm_head_kernel, the position-0 argmax fused, its logits never written) and the
    14-step rollout.  Algorithmic bytes: W once, hidden, the base rows of positions
    1..k-1 written, the first ids; the rollout's weights once (the low-rank head, rank
    projection, W_hh and prior stay on chip for the whole rollout, which is one launch
    at this shape); per step the base rows, the input-table rows and the ids.  The
    `library_lm_head` record times the same block with the library GEMM (hipBLASLt
    through torch.mm, as nn.Linear) followed by the position-0 argmax."""
    wl = pkg.synth.draft_block_workload(dev)
    B, k, d, V, E, G, r = 8, 15, 4096, 151936, 1024, 1024, 256
    steps = k - 1
    W = wl.W
    hiddens = wl.hiddens(3)
    n = 20
    cur = torch.cuda.current_stream(dev)

    def timed(fn):
        """Median over 7 timed runs of ``n`` calls, µs per call."""
        times = []
        for _ in range(7):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize(dev)
            e0.record(cur)
            for i in range(n):
                fn(i)
            e1.record(cur)
            torch.cuda.synchronize(dev)
            times.append(e0.elapsed_time(e1) / n)
        return replay_stats(times)["median"] * 1e3

    def make(lm_head):
        st = pkg.DeLSDraftStep(local_head=wl.head, lm_head_weight=W, batch_size=B, k_draft=k, vocab_size=V,
                               alpha_values=wl.alphas, beta_values=wl.betas, baseline_logits=wl.prior,
                               device=dev, lm_head=lm_head)
        for i in range(3):
            st(hiddens[i])
        torch.cuda.synchronize(dev)
        return st

    def block_of(st):
        def run(i):
            st.static_hidden.copy_(hiddens[i % 3])
            st.replay()
        return run

    weight_bytes = 2 * V * r + 2 * r * G + 2 * 3 * G * G + 2 * V           # low-rank head, A, W_hh, prior: once
    step_bytes = 2 * B * V + 2 * B * 3 * G + 12 * B                        # base rows, input-table rows, outputs

    # the default block: the hand-written LM head
    step = make("auto")
    assert step._fused_head, "the bench shape takes the hand-written LM head"
    us_block = timed(block_of(step))
    us_rollout = timed(lambda i: step.runner.replay())
    first = torch.empty(B, dtype=torch.int64, device=dev)
    first_sc = torch.empty(B, dtype=torch.float32, device=dev)
    us_head = timed(lambda i: pkg.lm_head(hiddens[i % 3].view(B * k, d), step._w_p,
                                          out=step.static_base.view(B * k, V), argmax_period=k, out_ids=first,
                                          out_score=first_sc))
    step.close()
    head_bytes = 2 * V * d + 2 * B * k * d + 2 * B * (k - 1) * V + 12 * B
    total = head_bytes + weight_bytes + steps * step_bytes

    # the same block with the library GEMM + row argmax
    lstep = make("library")
    us_lblock = timed(block_of(lstep))
    us_gemm = timed(lambda i: torch.mm(hiddens[i % 3].view(B * k, d), W.t(), out=lstep.static_base.view(B * k, V)))
    lstep.close()
    gemm_bytes = 2 * V * d + 2 * B * k * d + 2 * B * k * V
    ltotal = gemm_bytes + 2 * B * V + weight_bytes + steps * step_bytes
    return {"workload": "draft block: batch 8, block 16 (k_draft 15), d 4096, V 151936, local head G 1024 r 256",
            "lm_head": "lm_head_kernel (hand-written, position-0 argmax fused)",
            "us_per_block": us_block, "draft_tokens_per_s": B * k / (us_block * 1e-6),
            "us_lm_head": us_head, "lm_head_GBs": head_bytes / (us_head * 1e-6) / 1e9,
            "lm_head_hbm_frac": head_bytes / (us_head * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "us_rollout_14_steps": us_rollout,
            "algorithmic_bytes": total, "GBs": total / (us_block * 1e-6) / 1e9,
            "hbm_frac": total / (us_block * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "library_lm_head": {"lm_head": "hipBLASLt through torch.mm + argmax_rows_kernel",
                                "us_per_block": us_lblock, "us_lm_head_gemm": us_gemm,
                                "lm_head_GBs": gemm_bytes / (us_gemm * 1e-6) / 1e9,
                                "lm_head_hbm_frac": gemm_bytes / (us_gemm * 1e-6) / 1e9 / HBM_PEAK_GBS,
                                "algorithmic_bytes": ltotal,
                                "hbm_frac": ltotal / (us_lblock * 1e-6) / 1e9 / HBM_PEAK_GBS}}


def bench_batched_lm_head(pkg, dev, torch):
    """The target LM head that produces the M=512 record's base logits: 512 hidden rows
    (d 4096) against W [151936, 4096] bf16, bf16 logits [512, 151936] written --
    the library GEMM (hipBLASLt through torch.mm) and the hand-written lm_head_kernel
    (four row groups of 128, each re-streaming W).  Informative: it prices a kernel
    that would fuse this GEMM into the M=512 argmax (no base logits in HBM)."""
    M, d, V = 512, 4096, 151936
    g = torch.Generator(device=dev).manual_seed(512)
    W = (torch.randn(V, d, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    hid = torch.randn(M, d, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    Wp = pkg.pack_lm_head(W)
    cur = torch.cuda.current_stream(dev)

    def timed(fn, n=10):
        for _ in range(2):
            fn()
        times = []
        for _ in range(5):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize(dev)
            e0.record(cur)
            for _ in range(n):
                fn()
            e1.record(cur)
            torch.cuda.synchronize(dev)
            times.append(e0.elapsed_time(e1) / n)
        return replay_stats(times)["median"] * 1e3

    us_lib = timed(lambda: torch.mm(hid, W.t(), out=out))
    us_hw = timed(lambda: pkg.lm_head(hid, Wp, out=out))
    flops = 2.0 * M * d * V
    nbytes = 2 * V * d + 2 * M * d + 2 * M * V
    del W, Wp, out
    torch.cuda.empty_cache()
    return {"workload": "target LM head at M=512: hidden [512, 4096] . W[151936, 4096]^T, bf16 logits written",
            "us_library_gemm": us_lib, "library_TFLOPs": flops / (us_lib * 1e-6) / 1e12,
            "library_mfma_frac": flops / (us_lib * 1e-6) / 1e12 / BF16_MFMA_PEAK_TFLOPS,
            "us_hand_written": us_hw, "hand_written_TFLOPs": flops / (us_hw * 1e-6) / 1e12,
            "logits_bytes": 2 * M * V, "algorithmic_bytes": nbytes}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def time_cpu_path(fn, args, seconds, min_runs=20, warmup=3):
    """Median wall time (s) of ``fn(*args)`` after ``warmup`` calls: at least ``min_runs``
    timed calls, more while the time budget lasts (at most 200)."""
    for _ in range(warmup):
        fn(*args)
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        fn(*args)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_threads() -> int:
    """Threads for the CPU baseline: the share OMP_NUM_THREADS grants (16 per GPU on the
    GPU hosts), else every core."""
    env = os.environ.get("OMP_NUM_THREADS")
    return int(env) if env and env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def cpu_baseline(name, x0, seconds, gpu_ids=None):
    """The reference's CPU PyTorch path for one draft step of the workload, timed on this host.

    Timed: ``oracle.torch_eager.eager_step_bf16`` (the reference's eager bf16
    step: F.linear, bf16 combine, torch.argmax) and ``step_fp32`` (the same in
    fp32), median of >= 20 calls after 3 warm-ups with torch on ``cpu_threads()``
    threads.  ``value`` is the eager bf16 path's rows/s.  With ``gpu_ids`` (the
    device's ids for the same inputs) the agreement of each CPU path with them
    is reported too.
    """
    import torch

    from oracle import torch_eager

    threads = cpu_threads()
    torch.set_num_threads(threads)
    M = x0.shape["M"]
    args = (x0.h, x0.A, x0.B, x0.base, x0.prior, x0.alpha, x0.beta, x0.act)
    with torch.inference_mode():
        t_bf16, n_bf16 = time_cpu_path(torch_eager.eager_step_bf16, args, seconds / 2)
        t_f32, n_f32 = time_cpu_path(torch_eager.step_fp32, args, seconds / 2)
        ids_bf16 = torch_eager.eager_step_bf16(*args)
        ids_f32 = torch_eager.step_fp32(*args)
    out = {
        "value": M / t_bf16,
        "unit": "rows/s",
        "cores": threads,
        "kind": "port",
        "sample": f"median of {n_bf16} calls of one {name} draft step (M={M}: rank projection, low-rank logits, "
                  f"bf16 combine, argmax) through the reference's eager torch path restated in "
                  f"oracle/torch_eager.py; torch on {threads} threads of {os.cpu_count()} "
                  f"({cpu_model()})",
        "ms_per_step": t_bf16 * 1e3,
        "fp32_path": {"rows_per_s": M / t_f32, "ms_per_step": t_f32 * 1e3, "runs": n_f32},
    }
    if gpu_ids is not None:
        g = gpu_ids.cpu()
        out["gpu_id_agreement"] = {"vs_eager_bf16": float((g == ids_bf16).float().mean()),
                                   "vs_fp32": float((g == ids_f32).float().mean()), "rows": M}
    return out


def main():
    args = parse_args()
    if args.traffic_from:
        traffic_from(args)
        return
    if args.cpu_configs:
        import __graft_entry__

        pkg = __graft_entry__.load_package()
        for name in ("qwen3_4b_m16", "qwen3_8b_m16", "qwen3_8b_m512"):
            res = cpu_baseline(name, pkg.synth.config_inputs(name), args.cpu_seconds)
            print(json.dumps({"config": name, **res}), flush=True)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU per run: the fused argmax shards by rows or by "
                                   "vocabulary without collectives on the hot path; run with --gpus 1"}))
        sys.exit(2)
    import torch

    import __graft_entry__

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.ones(512 * 2**20 // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        print(json.dumps({"copy_calibration_bytes_per_copy": src.numel() * 4, "copies": 8}))
        return
    pkg = __graft_entry__.load_package()
    pkg._lib.load()

    rec, x0 = bench_workload(pkg, args.workload, args, dev, torch)
    traffic_all = {}
    if os.path.exists(args.traffic_file):
        try:
            with open(args.traffic_file) as fh:
                traffic_all = json.load(fh)
        except (OSError, ValueError):
            traffic_all = {}
    traffic = traffic_all.get(args.workload, {}).get("hbm_bytes_per_launch")
    one_launch = step_is_one_launch(args.workload, args.layout)
    if one_launch:
        # the step is the decode kernel: its bytes are the whole step's
        kernels = ROOFLINE_KERNELS[args.workload]
        roof_bytes, roof_us = rec["step_bytes"], rec["us_per_step"]
    else:
        kernels = ROOFLINE_KERNELS[args.workload] if args.layout == "packed" or args.workload == "qwen3_8b_m512" \
            else ROWMAJOR_M16_KERNELS
        roof_bytes, roof_us = rec["argmax_bytes"], rec["us_fused_argmax"]
        if args.layout != "packed":
            traffic = None       # the committed counters are of the packed run
    roof_gbs = roof_bytes / (roof_us * 1e-6) / 1e9
    out = {
        "metric": METRIC,
        "value": rec["rows_per_s"],
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": rec["us_per_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) h, N(0,0.02) A/B, N(0,3) base, permuted Zipf(1.1) log-prior; "
                f"{rec['sets']} rotating sets of {rec['set_MB']:.0f} MB)",
        "config": workload_desc(args.workload, x0, args.layout),
        "roofline": {
            "bound": "hbm",
            "kernel": " + ".join(kernels),
            "achieved": roof_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": roof_gbs / HBM_PEAK_GBS,
            "traffic": traffic,
            "algorithmic_bytes": roof_bytes,
            "us_per_launch": roof_us,
        },
        "timing": "median of 11 replays of one graph of K launches (HIP events on the launch stream); "
                  "spreads give p10/p90/min over the replays",
        "step": {k: rec[k] for k in ("us_per_step", "us_per_step_spread", "step_bytes", "step_GBs",
                                     "hbm_frac_step", "step_TFLOPs", "mfma_frac_step")},
        "fused_argmax_only": {"kernel": " + ".join(ROWMAJOR_M16_KERNELS if args.workload != "qwen3_8b_m512"
                                                   else ROOFLINE_KERNELS[args.workload]),
                              "us_per_launch": rec["us_fused_argmax"],
                              "us_per_launch_spread": rec["us_fused_argmax_spread"],
                              "algorithmic_bytes": rec["argmax_bytes"],
                              "GBs": rec["argmax_GBs"], "hbm_frac": rec["argmax_hbm_frac"]},
    }
    if args.also_m512 and args.workload != "qwen3_8b_m512":
        try:
            r512, _ = bench_workload(pkg, "qwen3_8b_m512", argparse.Namespace(**{**vars(args), "sets": 0,
                                                                                   "steps": min(args.steps, 100)}),
                                     dev, torch)
            out["m512"] = {k: r512[k] for k in ("rows_per_s", "us_per_step", "us_per_step_spread",
                                                "us_fused_argmax", "us_fused_argmax_spread", "argmax_GBs",
                                                "argmax_hbm_frac", "argmax_TFLOPs", "argmax_mfma_frac",
                                                "step_GBs", "hbm_frac_step", "step_TFLOPs", "mfma_frac_step")}
            out["m512"]["argmax_traffic"] = traffic_all.get("qwen3_8b_m512", {}).get("hbm_bytes_per_launch")
            out["m512"]["argmax_algorithmic_bytes"] = r512["argmax_bytes"]
        except Exception as e:  # informative record only
            out["m512"] = {"error": repr(e)}
        try:   # the same shape with fp32 base logits (the configuration runs bf16 ones, as the runtime does)
            r32, _ = bench_workload(pkg, "qwen3_8b_m512", argparse.Namespace(**{**vars(args), "sets": 0,
                                                                                  "steps": min(args.steps, 100)}),
                                    dev, torch, base_dtype=torch.float32)
            out["m512_fp32_base"] = {k: r32[k] for k in ("rows_per_s", "us_per_step", "us_per_step_spread",
                                                         "us_fused_argmax", "argmax_GBs", "argmax_hbm_frac",
                                                         "argmax_mfma_frac", "hbm_frac_step", "mfma_frac_step")}
            out["m512_fp32_base"]["argmax_algorithmic_bytes"] = r32["argmax_bytes"]
            out["m512_fp32_base"]["step_bytes"] = r32["step_bytes"]
        except Exception as e:  # informative record only
            out["m512_fp32_base"] = {"error": repr(e)}
    if args.also_draft_step and args.workload != "qwen3_8b_m512":
        try:
            out["draft_step"] = bench_draft_step(pkg, args, dev, torch)
        except Exception as e:  # informative record only
            out["draft_step"] = {"error": repr(e)}
    if args.also_batched_lm_head and args.also_m512 and args.workload != "qwen3_8b_m512":
        try:
            out["batched_lm_head"] = bench_batched_lm_head(pkg, dev, torch)
        except Exception as e:  # informative record only
            out["batched_lm_head"] = {"error": repr(e)}
    if args.also_domino and args.workload != "qwen3_8b_m512":
        try:
            out["domino"] = bench_domino(pkg, args, dev, torch)
        except Exception as e:  # informative record only
            out["domino"] = {"error": repr(e)}
    if args.also_fp8 and args.workload != "qwen3_8b_m512":
        try:
            out["fp8"] = bench_fp8(pkg, args.workload, args, dev, torch)
        except Exception as e:  # informative record only
            out["fp8"] = {"error": repr(e)}
        if args.also_m512:
            try:
                out["fp8_m512"] = bench_fp8(pkg, "qwen3_8b_m512", args, dev, torch)
            except Exception as e:  # informative record only
                out["fp8_m512"] = {"error": repr(e)}
    if args.cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.workload, x0, args.cpu_seconds, rec.get("ids_set0"))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
