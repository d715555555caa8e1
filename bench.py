"""Benchmark of one F rank's MoE layer on one MI355X.

Default workload: hidden 4096, moe_intermediate 2048, 256 experts of which this rank owns
[0, 64), top-8 uniform routing, one 16384-token dispatch, MXFP4 expert weights, bf16
activations at the boundary (MXFP8 inside). A "step" is one expert call over that job
(activation quantization, routing, grouped gate_up + SwiGLU, grouped down, finalize), with
inputs and packed weights resident in HBM.

Prints one JSON line: value = algorithmic TFLOPS (6 * H * I * Np per step, Np counted from
the generated ids), plus tokens/s, per-layer latency, per-stage times from HIP events on the
launch stream, the roofline of the dominant kernel (the gate_up GEMM) and the CPU baseline
(the fp32 CPU oracle on a bounded sample of the same workload). The default invocation also
runs the other workloads (the FP8-block layer, the one-GPU loop, the skewed job stream) as
child processes after its own timed steps and reports their headline numbers under
"other_workloads".
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "sgl-afd-plugin_amd")]

PEAK_TFLOPS = {"fp4": 10100.0, "fp8": 5000.0, "bf16": 2500.0}
PEAK_HBM_GBS = 8000.0
STAGES = ("hist_quant", "scatter", "gate_up", "down", "finalize")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=60)
    # the first ~25 layer calls after start-up run up to 45% slower while the GPU's clocks
    # settle: untimed calls before the warm-up steps, reported as settle_calls
    ap.add_argument("--settle-calls", type=int, default=40)
    ap.add_argument("--workload", default="layer", choices=["layer", "stream", "loop", "vendor"],
                    help="layer: one expert call per step (default); stream: the skewed job stream "
                    "from 2 replicas x 2 micro-batches through the F scheduler; loop: the one-GPU "
                    "A<->F loop with a shared expert, 2 micro-batches per layer; vendor: the vendor "
                    "library's dense fp8 GEMM (torch._scaled_mm, hipBLASLt) at the layer's padded "
                    "GEMM shapes, a ceiling to compare the grouped GEMMs with")
    ap.add_argument("--config", default="dsv4_rank", choices=["dsv4_rank", "ernie_fp8", "tiny"])
    ap.add_argument("--act", default=None, choices=["bf16"],
                    help="layer: the GEMMs' activation format (default: the weight format's fp8 "
                    "form; bf16 = W4A16 for MXFP4 weights)")
    ap.add_argument("--jobs", type=int, default=32, help="stream: jobs in the stream")
    ap.add_argument("--batch-tokens", type=int, default=32768,
                    help="stream: token capacity of the scheduler's batched expert calls in the "
                         "'batched' pass (the jobs of one poll packed into calls of at most this "
                         "many tokens)")
    ap.add_argument("--f-streams", type=int, default=None,
                    help="stream / loop: F streams the eager jobs alternate over (default: the loop's)")
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--cpu-baseline", type=int, default=1)
    ap.add_argument("--cpu-sample-tokens", type=int, default=4096)
    ap.add_argument("--cpu-sample-experts", type=int, default=16)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the timed steps, run a plain fp32 copy kernel (torch.neg) over MIB MiB "
                    "three times: the known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="no GPU: turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE, "
                    "WRITE_SIZE) of a --copy-calibration run into per-launch HBM bytes; writes --traffic-out")
    ap.add_argument("--stats-summary", metavar="KERNEL_STATS_CSV",
                    help="no GPU: print a rocprofv3 --stats kernel_stats.csv as a markdown table")
    ap.add_argument("--traffic-out", default=None)
    ap.add_argument("--others", default="auto", choices=["auto", "0", "1"],
                    help="layer: after the timed steps, run the other workloads (FP8-block layer, "
                    "loop, job stream) as child processes and report their numbers; auto = only "
                    "for the default report (the MXFP4 layer with the CPU baseline)")
    return ap.parse_args()


# the other workloads of the default report: name, bench.py flags, fields kept from its line
OTHER_WORKLOADS = (
    ("ernie_fp8_layer", ["--config", "ernie_fp8", "--cpu-baseline", "0", "--others", "0"],
     lambda d: {"tflops": d["value"], "ms_per_step": d["ms_per_step"], "stages_ms": d["stages_ms"],
                "gate_up_tflops": d["roofline"]["achieved"], "gate_up_frac_fp8": d["roofline"]["frac"]}),
    ("loop", ["--workload", "loop"],
     lambda d: {"layer_latency_ms": d["layer_latency_ms"], "layer_latency_ms_min": d["layer_latency_ms_min"],
                "chained_ms_per_layer": d["chained_ms_per_layer"],
                "tflops_routed_plus_shared": d["tflops_routed_plus_shared"]}),
    ("stream", ["--workload", "stream"],
     lambda d: {"batched_tflops": d["value"], "batched_ms": d["batched"]["ms"], "eager_ms": d["eager"]["ms"],
                "graphs_ms": d["graphs"]["ms"],
                "small_jobs": [{k: j[k] for k in ("tokens", "ms", "hbm_gbps")} for j in d["small_jobs"]]}),
)


def run_others() -> dict:
    """Each other workload in a child process of its own (its own warm-up, timing and memory),
    one after the other; a failed child is reported, not raised."""
    out = {"note": "each workload run as `python bench.py <flags>` in a child process after this "
                   "line's timed steps, with its own warm-up and timing"}
    for name, flags, keep in OTHER_WORKLOADS:
        t0 = time.monotonic()
        try:
            r = subprocess.run([sys.executable, os.path.abspath(__file__)] + flags, capture_output=True,
                               text=True, timeout=600, cwd=ROOT)
            lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
            if r.returncode != 0 or not lines:
                out[name] = {"flags": flags, "error": f"exit {r.returncode}", "stderr_tail": r.stderr[-400:]}
            else:
                out[name] = {"flags": flags, **keep(json.loads(lines[-1]))}
        except subprocess.TimeoutExpired:
            out[name] = {"flags": flags, "error": "timed out after 600 s"}
        out[name]["wall_s"] = round(time.monotonic() - t0, 1)
        print(f"[bench] {name}: {out[name]}", file=sys.stderr, flush=True)
    return out


TRAFFIC_DIR = os.path.join(ROOT, "profiles")


def _csv_rows(path):
    import csv

    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _short(name: str) -> str:
    n = name.replace("(anonymous namespace)::", "").replace("void ", "")
    if n.endswith(")"):
        n = n[: n.rfind("(")]
    return n[:90]


def pmc_summary(fetch_csv: str, write_csv: str, copy_mib: int, out_path) -> dict:
    """Average FETCH_SIZE / WRITE_SIZE (KiB per dispatch) per kernel, scaled so that the
    plain copy kernel of the same run reads and writes exactly ``copy_mib`` MiB."""
    per, copy_kib = {}, {}
    copy_grid = copy_mib * (1 << 20) // 4 // 4  # fp32 elements, 4 per lane of the copy kernel
    for which, path in (("fetch", fetch_csv), ("write", write_csv)):
        acc, cal = {}, []
        for r in _csv_rows(path):
            acc.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
            # the calibration copy: torch's neg over copy_mib MiB (other, smaller neg launches of
            # the input generators share its name, so it is told apart by its grid)
            if "neg_kernel" in r["Kernel_Name"] and int(r["Grid_Size"]) == copy_grid:
                cal.append(float(r["Counter_Value"]))
        if not cal:
            raise SystemExit(f"no {copy_mib} MiB copy kernel (torch neg, grid {copy_grid}) in {path}")
        per[which] = {k: sum(v) / len(v) for k, v in acc.items()}
        copy_kib[which] = sum(cal) / len(cal)
    known_kib = copy_mib * 1024.0
    f_fetch = known_kib / copy_kib["fetch"]
    f_write = known_kib / copy_kib["write"]
    kernels = {}
    for k in per["fetch"]:
        if "afd::" not in k:
            continue
        fb = per["fetch"][k] * f_fetch * 1024
        wb = per["write"].get(k, 0.0) * f_write * 1024
        kernels[_short(k)] = {"fetch_bytes": round(fb), "write_bytes": round(wb), "bytes": round(fb + wb)}
    out = {
        "copy_kernel_mib": copy_mib,
        "scale_fetch": round(f_fetch, 4),
        "scale_write": round(f_write, 4),
        "kernels": kernels,
    }
    if out_path:
        with open(out_path, "w") as f:
            json.dump(out, f, indent=1)
    return out


def stats_summary(path: str) -> str:
    rows = _csv_rows(path)
    lines = ["| kernel | calls | avg us | min us | max us | % |", "|---|---:|---:|---:|---:|---:|"]
    for r in rows:
        lines.append(
            f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
            f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |"
        )
    return "\n".join(lines)


def load_traffic(workload: str, kernel_key: str):
    """Per-launch HBM bytes of the dominant kernel from the committed PMC summary of this
    workload (profiles/traffic_<workload>.json), or None."""
    path = os.path.join(TRAFFIC_DIR, f"traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        data = json.load(f)
    hits = [v for k, v in data["kernels"].items() if kernel_key in k]
    return hits[0]["bytes"] if len(hits) == 1 else None


def cpu_baseline(shape, sample_tokens: int, sample_experts: int, act=None):
    """The fp32 CPU oracle on a bounded sample: the first ``sample_tokens`` tokens of the
    same seeded job, with only experts [0, sample_experts) treated as local (so the sample
    keeps the per-pair work of the full layer). 1 warm-up + 3 timed reps, median."""
    import numpy as np
    import torch

    from oracle import experts as OX
    from oracle import formats as F
    from sgl_asap_amd import workloads as W

    threads = len(os.sched_getaffinity(0))  # every host core this process may run on
    torch.set_num_threads(threads)
    gen = W.generator("cpu", 1)
    x, ids, w = W.job(shape, n=sample_tokens, seed=0, device="cpu")
    w13, w2 = W.expert_weights(sample_experts, shape.hidden, shape.inter, gen, "cpu")
    if shape.fmt == "mxfp4":
        c13, s13 = F.mx_quantize(w13.numpy(), "e2m1")
        c2, s2 = F.mx_quantize(w2.numpy(), "e2m1")
        w13d, w2d = F.mx_dequantize(c13, s13, "e2m1"), F.mx_dequantize(c2, s2, "e2m1")
        act_fp8 = "mxfp8"
    else:
        c13, s13 = F.fp8_block_quantize_2d(w13.numpy())
        c2, s2 = F.fp8_block_quantize_2d(w2.numpy())
        w13d, w2d = F.fp8_block_dequantize_2d(c13, s13), F.fp8_block_dequantize_2d(c2, s2)
        act_fp8 = "fp8_1x128"
    act = act or act_fp8
    ids_np, w_np = ids.numpy(), w.numpy()
    np_pairs = int(((ids_np >= 0) & (ids_np < sample_experts)).sum())
    times = []
    for rep in range(4):
        t0 = time.perf_counter()
        OX.moe_ffn(x, ids_np, w_np, w13d, w2d, 0, act=act)
        dt = time.perf_counter() - t0
        if rep:
            times.append(dt)
    t = statistics.median(times)
    tflops = 6.0 * shape.hidden * shape.inter * np_pairs / t / 1e12
    return {
        "value": round(tflops, 4),
        "unit": "TFLOPS",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"{sample_tokens} tokens of the same seeded job, experts [0,{sample_experts}) local "
            f"({np_pairs} pairs), fp32 torch CPU oracle ({act} activations) incl. act quant/routing/finalize; "
            f"median of 3 reps = {t * 1e3:.1f} ms"
        ),
    }


def _mxfp4_layer(W, shape, dev, n_max, seed=1):
    """One layer of packed MXFP4 local experts of ``shape`` (weights ~ N(0, 0.02))."""
    import torch

    from sgl_asap_amd.moe.experts import AfdExperts, pack_mxfp4_experts

    w13, w2 = W.expert_weights(shape.num_local, shape.hidden, shape.inter, W.generator(dev, seed), dev)
    weights = pack_mxfp4_experts(w13, w2, device=dev)
    del w13, w2
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return AfdExperts(shape.num_experts, shape.top_k, 0, shape.local, weights, n_max=n_max)


def _f_streams(args) -> dict:
    return {} if getattr(args, "f_streams", None) is None else {"f_streams": args.f_streams}


def small_jobs(W, shape, dev, sizes=(256, 512, 1024, 2048)) -> list:
    """Single small jobs of the stream's shape through the eager expert call: at these sizes
    the layer is bound by streaming the touched experts' weights from HBM. Compulsory bytes =
    weights of the local experts with at least one pair + x + out + ids + w."""
    import torch

    from sgl_asap_amd.moe.topk import StandardTopKOutput

    experts = _mxfp4_layer(W, shape, dev, max(sizes))
    per_expert = (experts.weights.w13.numel() + experts.weights.w2.numel()) // shape.num_local
    rows = []
    for n in sizes:
        x, ids, w = W.job(shape, n=n, seed=900 + n, device=dev)
        topk = StandardTopKOutput(w.to(torch.float32), ids.to(torch.int32))
        rel = ids - shape.local.start
        touched = int(torch.unique(rel[(rel >= 0) & (rel < shape.num_local)]).numel())
        nbytes = touched * per_expert + n * shape.hidden * 4 + n * shape.top_k * 8
        for _ in range(20):
            experts(x, topk)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            experts(x, topk)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 20
        rows.append({"tokens": n, "experts_touched": touched, "ms": round(ms, 4),
                     "compulsory_bytes": nbytes, "hbm_gbps": round(nbytes / (ms * 1e-3) / 1e9, 1)})
    del experts
    torch.cuda.empty_cache()
    return rows


def bench_stream(args) -> dict:
    """The skewed job stream: Zipf(1.2) routing, job sizes log-uniform in [256, 16384], jobs
    arriving from 2 A replicas x 2 micro-batches (round robin) through the one-GPU transport
    into the F scheduler, served three ways: with one eager expert call per job, with HIP
    graphs for every power-of-two bucket up to 16384 tokens, and with the jobs of each poll
    packed into batched expert calls of up to --batch-tokens tokens (the value). Timed: first
    send to the last reply landing, after one untimed pass of the same stream, which also
    collects the per-call GPU times (job_clock)."""
    import torch

    from sgl_asap_amd import workloads as W
    from sgl_asap_amd.loop import OneGpuAfd

    shape = W.SHAPES["dsv4_zipf"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n_max = 16384
    sizes = W.job_sizes(args.jobs, 256, n_max, seed=0)
    jobs = []
    for j, n in enumerate(sizes):
        x, ids, w = W.job(shape, n=n, seed=100 + j, device=dev)
        jobs.append((x, ids.to(torch.int32).contiguous(), w.to(torch.float32).contiguous()))
    pairs = sum(W.pair_count(ids, shape.local) for _, ids, _ in jobs)
    flops = W.flops(shape.hidden, shape.inter, pairs)
    tokens = sum(sizes)
    order = [(r, mb) for r in range(2) for mb in range(2)]
    out = {
        "metric": "MoE-layer TFLOPS + tokens/s, skewed job stream (2 replicas x 2 micro-batches), 1 MI355X",
        "unit": "TFLOPS",
        "n_gpus": 1,
        "higher_is_better": True,
        "dtype": "mxfp4xmxfp8",
        "data": "synthetic (seeded N(0,1) tokens, Zipf(1.2) routing, N(0,0.02) expert weights, random-init)",
        "config": {
            "workload": f"dsv4_zipf job stream: one F rank, H={shape.hidden} I={shape.inter}, "
            f"{shape.num_local} local of {shape.num_experts} experts, top-{shape.top_k}, {len(sizes)} jobs "
            f"of logU[256,16384] tokens ({tokens} tokens, {pairs} local pairs)",
            "job_tokens": sizes,
        },
    }
    for mode, graph_max, batch in (("graphs", n_max, 0), ("eager", 0, 0), ("batched", 0, args.batch_tokens)):
        experts = {0: _mxfp4_layer(W, shape, dev, n_max)}
        t0 = time.perf_counter()
        afd = OneGpuAfd(experts, n_max=n_max, slots=2, replicas=2, graph_max_tokens=graph_max, timing=True,
                        batch_tokens=batch, **_f_streams(args))
        setup_s = time.perf_counter() - t0
        sends = [torch.cuda.Stream() for _ in range(2)]
        main = torch.cuda.current_stream()

        def run():
            for s in sends:
                s.wait_stream(main)
            for base in range(0, len(jobs), len(order)):
                tickets = []
                for k, (r, mb) in enumerate(order):
                    if base + k < len(jobs):
                        x, ids, w = jobs[base + k]
                        tickets.append((r, afd.channels[r].send(0, mb, x.data_ptr(), ids.data_ptr(),
                                                                  w.data_ptr(), x.shape[0], sends[r])))
                afd.scheduler.serve_pending()
                for r, t in tickets:
                    afd.channels[r].wait(t, main)

        run()  # untimed, with the per-job clock (two event records per job)
        torch.cuda.synchronize()
        clock, afd.scheduler.clock = afd.scheduler.clock, None  # the timed pass records nothing
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        h0 = time.perf_counter()
        e0.record(main)
        run()
        e1.record(main)
        host_ms = (time.perf_counter() - h0) * 1e3
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
        afd.scheduler.clock = clock
        out[mode] = {
            "ms": round(ms, 3),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
            "tokens_per_s": round(tokens / (ms * 1e-3), 1),
            "host_enqueue_ms": round(host_ms, 3),
            "setup_s": round(setup_s, 2),
            "f_streams": len(afd.scheduler.streams),
            "expert_calls_per_pass": afd.scheduler.expert_calls // 2,
            "batch_tokens": batch,
            "jobs_per_bucket": {str(b): v["jobs"] for b, v in afd.scheduler.clock.summary().items()},
            "job_clock": afd.scheduler.clock.summary(),
        }
        afd.close()
        del experts, afd
        torch.cuda.empty_cache()
    out["small_jobs"] = small_jobs(W, shape, dev)
    # value: the F scheduler serving the jobs of each poll in batched expert calls (each job's
    # output identical to its own call); one eager call per job (the reference's way) and the
    # replays of the captured graphs are timed beside it
    out["value_pass"] = "batched"
    out["value"] = out["batched"]["tflops"]
    out["ms_per_step"] = out["batched"]["ms"]
    out["tokens_per_s"] = out["batched"]["tokens_per_s"]
    return out


def bench_loop(args) -> dict:
    """The one-GPU A<->F loop at W4A8 with a bf16 shared expert (intermediate 1536): per layer
    two micro-batches of 8192 tokens (Zipf(1.2) routing) are dispatched on slots 0/1 (arena
    copies + doorbells on the A send stream), the F scheduler parks its stream on the
    doorbells and runs the experts (one eager expert call per job; with HIP graph replays
    for comparison), the shared expert runs on the A compute
    stream meanwhile, and the combine adds the routed partial sums and the shared output.
    Per-layer latency: from before the first copy to the last combine's output."""
    import torch

    from sgl_asap_amd import workloads as W
    from sgl_asap_amd.loop import OneGpuAfd
    from sgl_asap_amd.moe.layer import AsapMoE
    from sgl_asap_amd.moe.shared import SharedExpertMLP
    from sgl_asap_amd.moe.topk import StandardTopKOutput

    shape = W.SHAPES["dsv4_zipf"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n, shared_i = 8192, 1536
    experts = {0: _mxfp4_layer(W, shape, dev, n)}
    shared = SharedExpertMLP.random(shape.hidden, shared_i, W.generator(dev, 2), dev)

    mbs = []
    for m in range(2):
        x, ids, w = W.job(shape, n=n, seed=200 + m, device=dev)
        mbs.append((x, StandardTopKOutput(w.to(torch.float32), ids.to(torch.int32))))
    pairs = sum(W.pair_count(t.topk_ids, shape.local) for _, t in mbs)
    routed_flops = W.flops(shape.hidden, shape.inter, pairs)
    shared_flops = 2 * 6 * shape.hidden * shared_i * n
    layer = AsapMoE(shape.num_experts, shape.hidden, shape.inter, 0, top_k=shape.top_k)
    main = torch.cuda.current_stream()

    def measure(act, graphs=False):
        afd = OneGpuAfd(experts, n_max=n, slots=2, graph_max_tokens=n if graphs else 0, act=act,
                        **_f_streams(args))

        def step():
            d = [layer.dispatcher.dispatch(x, t, micro_batch=m) for m, (x, t) in enumerate(mbs)]
            afd.scheduler.serve_pending()
            s = [shared(x) for x, _ in mbs]
            return [layer.dispatcher.combine(d[m], s[m]) for m in range(2)]

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        lat = []
        for _ in range(args.steps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(main)
            step()
            e1.record(main)
            torch.cuda.synchronize()
            lat.append(e0.elapsed_time(e1))
        # Chained layers: each step's micro-batch m dispatches the previous step's combine
        # output of m (the data dependency of consecutive MoE layers; attention left out), with
        # no host synchronization between the steps, as a serving loop runs them. The host
        # enqueues ahead, so its latency hides behind the GPU work of the earlier layers.
        xs = [x for x, _ in mbs]
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(main)
        for _ in range(args.steps):
            d = [layer.dispatcher.dispatch(xs[m], mbs[m][1], micro_batch=m) for m in range(2)]
            afd.scheduler.serve_pending()
            s = [shared(x) for x in xs]
            xs = [layer.dispatcher.combine(d[m], s[m]) for m in range(2)]
        e1.record(main)
        torch.cuda.synchronize()
        chained.append(e0.elapsed_time(e1) / args.steps)
        streams_used.append(len(afd.scheduler.streams))
        afd.close()
        return lat

    streams_used, chained = [], []
    # activations on the wire: bf16 (the reference's layout), then MXFP8 (A quantizes before
    # the copy; bit-identical outputs, half the copy bytes, no quantizer on the F side)
    lat_fp8 = measure("mxfp8")
    lat = measure("bf16")
    lat_graphs = measure("bf16", graphs=True)
    # the A-side combine alone at this size: 1 F part + the shared output -> bf16
    from sgl_asap_amd.moe.dispatcher import combine_parts

    part = torch.randn(n, shape.hidden, device=dev).to(torch.bfloat16)
    sh = torch.randn(n, shape.hidden, device=dev).to(torch.bfloat16)
    for _ in range(5):
        combine_parts([part.data_ptr()], sh, n, shape.hidden, dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        combine_parts([part.data_ptr()], sh, n, shape.hidden, dev)
    e1.record()
    torch.cuda.synchronize()
    comb_ms = e0.elapsed_time(e1) / 20
    comb_bytes = 3 * n * shape.hidden * 2
    ms = statistics.median(lat)
    ms_fp8 = statistics.median(lat_fp8)
    return {
        "metric": "per-layer latency of the one-GPU AFD loop (W4A8 + bf16 shared expert), 1 MI355X",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "dtype": "mxfp4xmxfp8 routed, bf16 shared",
        "data": "synthetic (seeded N(0,1) tokens, Zipf(1.2) routing, N(0,0.02) weights, random-init)",
        "config": {
            "workload": f"dsv4_zipf loop: 2 micro-batches x {n} tokens, H={shape.hidden} I={shape.inter}, "
            f"{shape.num_local} local of {shape.num_experts} experts, top-{shape.top_k}, shared expert I={shared_i} bf16",
            "local_pairs": pairs,
            "f_streams": streams_used[0],
        },
        "layer_latency_ms": round(ms, 4),
        "layer_latency_ms_min": round(min(lat), 4),
        # chained: ms per layer over the timed steps run as consecutive layers (each one's
        # inputs are the previous one's outputs, no synchronization between them); in the
        # order of the measures below (fp8 wire, bf16 wire, bf16 with graph replays)
        "chained_ms_per_layer": {"mxfp8": round(chained[0], 4), "bf16": round(chained[1], 4),
                                 "bf16_graphs": round(chained[2], 4)},
        "tokens_per_s": round(2 * n / (ms * 1e-3), 1),
        "tflops_routed_plus_shared": round((routed_flops + shared_flops) / (ms * 1e-3) / 1e12, 2),
        "combine": {"ms": round(comb_ms, 4), "bytes": comb_bytes,
                    "hbm_gbps": round(comb_bytes / (comb_ms * 1e-3) / 1e9, 1)},
        "wire": "bf16",
        "fp8_wire": {"act": "mxfp8", "layer_latency_ms": round(ms_fp8, 4),
                     "layer_latency_ms_min": round(min(lat_fp8), 4),
                     "tokens_per_s": round(2 * n / (ms_fp8 * 1e-3), 1)},
        "graphs": {"wire": "bf16", "layer_latency_ms": round(statistics.median(lat_graphs), 4),
                   "layer_latency_ms_min": round(min(lat_graphs), 4)},
    }


def bench_vendor(args) -> dict:
    """The vendor library's dense e4m3 x e4m3 GEMM (torch._scaled_mm on hipBLASLt, bf16 out,
    per-tensor scales) at the config's two GEMM shapes with the expert call's padded row count
    (every local expert's rows rounded up to 128): the same MFMA rate as the grouped W4A8 and
    FP8 GEMMs, without their gather, routing and epilogues. With ``--act bf16`` the dense bf16 x
    bf16 GEMM (torch.mm on hipBLASLt), the MFMA rate of the bf16-activation GEMMs."""
    import torch

    from sgl_asap_amd import workloads as W

    shape = W.SHAPES[args.config]
    n = args.tokens or shape.tokens
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _, ids, _ = W.job(shape, n=n, seed=0, device=dev)
    lo, hi = shape.local.start, shape.local.stop
    local = ids[(ids >= lo) & (ids < hi)] - lo
    counts = torch.bincount(local.flatten().long(), minlength=hi - lo)
    padded = int(((counts + 127) // 128 * 128).sum())
    out = {}
    bf16 = args.act == "bf16"
    for name, (m, nn, k) in (("gate_up", (padded, 2 * shape.inter, shape.hidden)),
                             ("down", (padded, shape.hidden, shape.inter))):
        dt = torch.bfloat16 if bf16 else torch.float8_e4m3fn
        a = torch.randn(m, k, device=dev).to(dt)
        b = torch.randn(nn, k, device=dev).to(dt)
        one = torch.ones((), device=dev)

        def mm():
            if bf16:
                return torch.mm(a, b.t())
            return torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)

        for _ in range(args.warmup):
            mm()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            mm()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / args.steps
        out[name] = {"m": m, "n": nn, "k": k, "us": round(us, 1), "tflops": round(2 * m * nn * k / us / 1e6, 1)}
        del a, b
    return {
        "metric": f"dense {'bf16' if bf16 else 'fp8'} GEMM throughput of the vendor library at the expert call's GEMM shapes",
        "value": out["gate_up"]["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "higher_is_better": True,
        "dtype": "bf16 x bf16 -> bf16" if bf16 else "e4m3 x e4m3 -> bf16",
        "data": "synthetic (N(0,1) operands)",
        "config": {"workload": f"{args.config}: {padded} padded rows "
                               f"({'torch.mm' if bf16 else 'torch._scaled_mm'}, hipBLASLt)"},
        "gemms": out,
    }


def main():
    args = parse()
    if args.stats_summary:
        print(stats_summary(args.stats_summary))
        return
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary, args.copy_calibration or 1024, args.traffic_out), indent=1))
        return
    if args.gpus != 1:
        print(
            f"bench.py measures one F rank's share of the experts on one GPU; --gpus {args.gpus} "
            "is not supported (the path shards by expert range, one F rank per GPU, with no "
            "collectives: run one process per GPU)",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    if args.workload == "stream":
        print(json.dumps(bench_stream(args)), flush=True)
        return
    if args.workload == "loop":
        print(json.dumps(bench_loop(args)), flush=True)
        return
    if args.workload == "vendor":
        print(json.dumps(bench_vendor(args)), flush=True)
        return

    from sgl_asap_amd import _lib
    from sgl_asap_amd import workloads as W
    from sgl_asap_amd.moe.experts import AfdExperts, pack_fp8_block_experts, pack_mxfp4_experts

    shape = W.SHAPES[args.config]
    n = args.tokens or shape.tokens
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    x, ids, w = W.job(shape, n=n, seed=0, device=dev)
    gen = W.generator(dev, 1)
    w13, w2 = W.expert_weights(shape.num_local, shape.hidden, shape.inter, gen, dev)
    pack = pack_mxfp4_experts if shape.fmt == "mxfp4" else pack_fp8_block_experts
    weights = pack(w13, w2, device=dev)
    del w13, w2
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    experts = AfdExperts(shape.num_experts, shape.top_k, 0, shape.local, weights, n_max=n, act_format=args.act)
    a16 = experts.act_format == "bf16"
    np_pairs = W.pair_count(ids, shape.local)
    flops = W.flops(shape.hidden, shape.inter, np_pairs)
    gate_up_flops = 4 * shape.hidden * shape.inter * np_pairs

    stream = torch.cuda.current_stream()
    out = torch.empty(n, shape.hidden, dtype=torch.bfloat16, device=dev)
    ws = experts.workspace()
    cfg, wst = experts.cfg, experts._wstruct
    ids32, w32 = ids.to(torch.int32).contiguous(), w.to(torch.float32).contiguous()

    def step(evs=None):
        """One expert call: the product entry point, or with evs the profiled one, which
        records the stage boundaries given (None entries skipped) on the stream, a few us each."""
        if evs is None:
            _lib.call(
                "afd_moe_ffn", ctypes.byref(cfg), ctypes.byref(wst), x.data_ptr(), ids32.data_ptr(),
                w32.data_ptr(), n, ws.data_ptr(), ws.numel(), out.data_ptr(), stream.cuda_stream,
            )
            return
        arr = (ctypes.c_void_p * 6)(*[e.cuda_event if e is not None else None for e in evs])
        _lib.call(
            "afd_moe_ffn_profiled", ctypes.byref(cfg), ctypes.byref(wst), x.data_ptr(), ids32.data_ptr(),
            w32.data_ptr(), n, ws.data_ptr(), ws.numel(), out.data_ptr(), stream.cuda_stream, arr,
        )

    for _ in range(args.settle_calls + args.warmup):
        step()
    torch.cuda.synchronize()

    # per-step stage events (recorded once first so their HIP handles exist)
    ev_sets = []
    for _ in range(args.steps):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        for e in evs:
            e.record(stream)
        ev_sets.append(evs)
    torch.cuda.synchronize()

    # the timed steps: the product entry point, nothing else on the stream
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for _ in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    ms = t_start.elapsed_time(t_end) / args.steps
    # the dominant kernel's duration, live, on the stream it runs on: a second timed pass of
    # the same steps with events around the gate_up launch only (each record leaves a ~6 us
    # gap before the next launch, so they stay out of the steps timed above)
    gu_sets = []
    for _ in range(args.steps):
        evs = [None, None, torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True), None, None]
        evs[2].record(stream)
        evs[3].record(stream)
        gu_sets.append(evs)
    torch.cuda.synchronize()
    for k in range(args.steps):
        step(gu_sets[k])
    torch.cuda.synchronize()
    gu_ms = sum(e[2].elapsed_time(e[3]) for e in gu_sets) / args.steps
    # stage breakdown: a second pass of the same steps through the profiled entry point
    for k in range(args.steps):
        step(ev_sets[k])
    torch.cuda.synchronize()

    stage_ms = {s: [] for s in STAGES}
    for evs in ev_sets:
        for i, s in enumerate(STAGES):
            stage_ms[s].append(evs[i].elapsed_time(evs[i + 1]))
    stage_avg = {s: round(sum(v) / len(v), 5) for s, v in stage_ms.items()}

    if args.copy_calibration:  # known-size reference kernel for the PMC byte counters
        src = torch.ones(args.copy_calibration << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    tflops = flops / (ms * 1e-3) / 1e12
    # algorithmic bytes of the streaming phases (their own tensors' reads + writes)
    k, h = shape.top_k, shape.hidden
    xs_bytes = n * h // 32 if shape.fmt == "mxfp4" else n * h // 128 * 4
    phase_bytes = {
        # ids; x in; codes + scales out (bf16 activations: the histogram of the ids only)
        "hist_quant": n * k * 4 if a16 else n * k * 4 + n * h * 2 + n * h + xs_bytes,
        "scatter": n * k * 4 + n * k * 4 + np_pairs * 4,  # ids in; pair_pos, sorted pairs out
        "finalize": np_pairs * h * 2 + n * k * 8 + n * h * 2,  # y rows, pair_pos + w; out
    }
    phase_gbps = {s: round(b / (stage_avg[s] * 1e-3) / 1e9, 1) for s, b in phase_bytes.items()}
    gu_tflops = gate_up_flops / (gu_ms * 1e-3) / 1e12
    issued = "bf16" if a16 else "fp8"
    wfmt = 0 if shape.fmt == "mxfp4" else 1
    if a16:
        kernel, kernel_key = f"a16_gemm_kernel<{shape.fmt}, gate_up>", f"a16_gemm_kernel<{wfmt}, 0"
    elif shape.fmt == "mxfp4":
        kernel, kernel_key = "mx_gemm_kernel<gate_up>", "mx_gemm_kernel<0"
    else:
        kernel, kernel_key = "fp8_gemm_kernel<gate_up>", "fp8_gemm_kernel<0"
    traffic_name = shape.name + ("_a16" if a16 else "")
    result = {
        "metric": "MoE-layer TFLOPS + tokens/s at 16k-token dispatch, 1 MI355X; MFMA util %",
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_calls": args.settle_calls,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("mxfp4xbf16" if a16 else "mxfp4xmxfp8") if shape.fmt == "mxfp4"
        else ("fp8(block)xbf16" if a16 else "fp8xfp8(block)"),
        "data": "synthetic (seeded N(0,1) tokens, N(0,0.02) expert weights, random-init)",
        "config": {
            "workload": f"{shape.name}: one F rank, H={shape.hidden} I={shape.inter}, "
            f"{shape.num_local} local of {shape.num_experts} experts, top-{shape.top_k}, "
            f"{'uniform' if shape.zipf is None else f'Zipf({shape.zipf})'} routing, {n} tokens, {shape.fmt} weights, "
            f"{experts.act_format} activations",
            "tokens": n,
            "local_pairs": np_pairs,
            "algorithmic_tflop": round(flops / 1e12, 4),
        },
        "tokens_per_s": round(n / (ms * 1e-3), 1),
        "layer_latency_ms": round(ms, 4),
        "mfma_util_vs_fp4_peak": round(tflops / PEAK_TFLOPS["fp4"], 4),
        "mfma_util_vs_issued_peak": round(tflops / PEAK_TFLOPS[issued], 4),
        "stages_ms": stage_avg,
        "phase_bytes": phase_bytes,
        "phase_hbm_gbps": phase_gbps,
        "stages_note": "from a third pass of the same steps through afd_moe_ffn_profiled with all "
        "six stage events; the timed steps call afd_moe_ffn with no events, and roofline.kernel_ms "
        "comes from a second pass with events around gate_up only. hist_quant: the expert "
        "histogram and the activation quantization in one launch; scatter: the router's scan and "
        "pair scatter",
        "roofline": {
            "kernel": f"grouped gate_up GEMM + SwiGLU ({kernel})",
            "bound": "mfma",
            "achieved": round(gu_tflops, 2),
            "kernel_ms": round(gu_ms, 5),
            "peak": PEAK_TFLOPS["fp4"] if shape.fmt == "mxfp4" else PEAK_TFLOPS["fp8"],
            "unit": "TFLOP/s",
            "frac": round(gu_tflops / (PEAK_TFLOPS["fp4"] if shape.fmt == "mxfp4" else PEAK_TFLOPS["fp8"]), 4),
            "frac_vs_issued_format_peak": round(gu_tflops / PEAK_TFLOPS[issued], 4),
            "traffic": load_traffic(traffic_name, kernel_key),
        },
    }
    if args.cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(shape, min(args.cpu_sample_tokens, n), min(args.cpu_sample_experts, shape.num_local),
                                              experts.act_format)
    default_report = (args.cpu_baseline and args.config == "dsv4_rank" and args.act is None and args.tokens is None
                      and not args.copy_calibration)
    if args.others == "1" or (args.others == "auto" and default_report):
        del experts, weights, ws, x, out
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        result["other_workloads"] = run_others()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
