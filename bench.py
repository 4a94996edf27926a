#!/usr/bin/env python3
"""W4A16 fused dequant + linear benchmark on one MI355X.

Workload (the 12B-like decode linears at M=1): one
step is one decode layer's worth of W4A16 linears on one token --
q 3840->4096, k 3840->2048, v 3840->2048, o 4096->3840, gate/up fused
3840->30720, down 15360->3840 -- with bf16 activations in and bf16 out.
Consecutive steps walk distinct weight sets (as consecutive layers do), and the
sets together exceed 512 MB so that the 256 MB MALL cannot hold them: every
step streams its weights from HBM.

value = algorithmic bytes per step / time per step (GB/s), where the bytes of a
linear are N*K/2 (packed) + 2*N*K/32 (scales) + 2*M*K (x) + 2*M*N (y).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--all]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "gemma4-zml-probe_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "W4A16 GEMV achieved HBM GB/s (% of peak) at M=1; TFLOP/s at M=64"
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, published
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, published
ROTATE_BYTES = 600 * 2**20     # > 512 MB working set

LAYER_12B = [  # name, K, N
    ("q", 3840, 4096), ("k", 3840, 2048), ("v", 3840, 2048), ("o", 4096, 3840),
    ("gate_up", 3840, 30720), ("down", 15360, 3840),
]
DOMINANT = "gate_up"
DOMINANT_KERNEL = "w4k::gemv_fast_kernel<1, 2, 1, true, 4, true, true, 1, false, false>"  # the launch the M=1 plan picks for 12B gate/up
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_fast_12b_gateup_m1_pmc.md")


def lin_bytes(M: int, K: int, N: int) -> int:
    return N * K // 2 + 2 * N * (K // 32) + 2 * M * K + 2 * M * N


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_info() -> dict:
    """What __graft_entry__.build() recorded next to libw4a16.so (git commit of the
    sources, dirty flag, build time, compiler flags), or {}."""
    try:
        with open(os.path.join(ROOT, "gemma4-zml-probe_amd", "build_info.json")) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def gpu_clocks() -> str:
    """Current / highest shader (sclk) and memory (mclk) clock levels of the first GPU,
    from its sysfs DPM tables ('*' marks the current level), or '?'."""
    import glob
    for dev in sorted(glob.glob("/sys/class/drm/card*/device")):
        out = []
        for name in ("pp_dpm_sclk", "pp_dpm_mclk"):
            try:
                with open(os.path.join(dev, name)) as f:
                    lines = [ln.strip() for ln in f if ln.strip()]
            except OSError:
                break
            cur = [ln.split(":", 1)[1].replace("*", "").strip() for ln in lines if ln.endswith("*")]
            top = lines[-1].split(":", 1)[1].replace("*", "").strip() if lines else "?"
            out.append(f"{name[-4:]}={cur[0] if cur else '?'}(max {top})")
        if len(out) == 2:
            return ",".join(out)
    return "?"


def read_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    --pmc summary (line 'traffic_bytes_per_launch: <int>'), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1].strip()))
    except OSError:
        pass
    return None


def make_set(torch, o, K, N, seed):
    """Synthetic packed weights generated on the GPU: iid uniform 32-bit words
    are iid uniform nibbles, i.e. q ~ U{-8..7}; scales bf16(|N(0,1)| * 0.02)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    pkd = torch.randint(-2**31, 2**31, (N, K // 8), generator=g, device="cuda", dtype=torch.int64).to(torch.int32)
    scd = (torch.randn((N, K // 32), generator=g, device="cuda").abs() * 0.02).to(torch.bfloat16)
    return pkd, scd


def synth_x_dev(torch, o, M, K, seed=None):
    """Activations bf16(N(0,1)) [M, K] drawn on the GPU (seed 2000 + M by default)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(2000 + M if seed is None else seed)
    return torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)


def graph_of(torch, fn):
    """Capture fn() (a sequence of libw4a16 launches on the current stream) in a HIP graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # one eager pass on the side stream before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def steady(torch, g, seconds=0.3, min_replays=2):
    """Replay g untimed until `seconds` of wall time have passed: the first
    milliseconds of a heavy run are slower (clock ramp-up) by up to ~15 %."""
    t0 = time.perf_counter()
    n = 0
    while n < min_replays or time.perf_counter() - t0 < seconds:
        g.replay()
        torch.cuda.synchronize()
        n += 1


def time_graph(torch, g, replays, warmup=2):
    steady(torch, g, min_replays=warmup)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3


def time_config(torch, w4a16, o, M, K, N, launches=None):
    """Average duration of one linear launch: a HIP graph of back-to-back launches
    rotating over weight sets larger than the MALL, timed with events around its
    replays (no host launch overhead between kernels)."""
    nbytes = lin_bytes(M, K, N)
    nsets = max(2, -(-ROTATE_BYTES // (N * K // 2 + N * K // 16)))
    sets = [make_set(torch, o, K, N, 7000 + i) for i in range(nsets)]
    x = synth_x_dev(torch, o, M, K)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    if launches is None:
        launches = nsets * max(1, -(-40 // nsets)) if M < 512 else nsets
    def run():
        for i in range(launches):
            pk, sc = sets[i % nsets]
            w4a16.linear(x, pk, sc, out=y)
    g = graph_of(torch, run)
    reps = 5 if M < 512 else 2
    t = time_graph(torch, g, reps) / (reps * launches)
    del g, sets
    torch.cuda.empty_cache()
    return {"M": M, "K": K, "N": N, "bytes": nbytes, "flops": 2 * M * N * K, "us": t * 1e6,
            "GBps": nbytes / t / 1e9, "hbm_frac": nbytes / t / 1e9 / PEAK_HBM_GBS,
            "TFLOPs": 2 * M * N * K / t / 1e12, "mfma_frac": 2 * M * N * K / t / 1e12 / PEAK_BF16_TFLOPS,
            "sets": nsets, "launches": launches}


def cpu_threads() -> int:
    """Threads for the CPU legs: the CPUs this process may run on (its affinity set),
    capped by OMP_NUM_THREADS when set -- the GPU box gives a job a share of the
    host's cores (16 per GPU) while os.cpu_count() reports the whole host."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "?"


# BASELINE.json configs for the CPU legs: name -> list of (M, K, N) linears per run
CPU_CONFIGS = {
    "C1": [(1, 1536, 6144)],
    "C2": [(1, K, N) for K, N in [(1536, 2048), (1536, 256), (1536, 256), (2048, 1536), (1536, 12288), (6144, 1536)]],
    "C3": [(1, K, N) for _, K, N in LAYER_12B],
    **{f"C4_M{M}": [(M, K, N) for _, K, N in LAYER_12B] for M in (8, 16, 32, 64)},
    "C5": [(2048, 3840, 30720), (2048, 15360, 3840)],
}


def cpu_config(name: str, budget_s: float, min_runs: int = 10, warmup: int = 3):
    """Both CPU legs of one config on the host cores: the
    reference's dequant + matmul per call (oracle/cpu_path.py), and the matmul alone on
    weights dequantized beforehand; median, p10 and p90 over >= min_runs runs (fewer
    when one run exceeds budget_s / min_runs, never fewer than 3) after `warmup` runs."""
    import torch
    from oracle import cpu_path

    torch.set_num_threads(cpu_threads())
    g = torch.Generator()
    g.manual_seed(8000)
    mats = []
    for M, K, N in CPU_CONFIGS[name]:
        pk = torch.randint(-2**31, 2**31, (N, K // 8), generator=g, dtype=torch.int64).to(torch.int32)
        sc = (torch.randn((N, K // 32), generator=g).abs() * 0.02).to(torch.bfloat16)
        x = torch.randn((M, K), generator=g).to(torch.bfloat16)
        mats.append((pk, sc, x))
    nbytes = sum(lin_bytes(M, K, N) for M, K, N in CPU_CONFIGS[name])
    flops = sum(2 * M * N * K for M, K, N in CPU_CONFIGS[name])

    def dq_mm():
        for pk, sc, x in mats:
            cpu_path.linear(x, pk, sc).to(torch.bfloat16)

    wf = None

    def mm():
        for (pk, sc, x), w in zip(mats, wf):
            (x.to(torch.float32) @ w.t()).to(torch.bfloat16)

    def measure(fn):
        for _ in range(warmup):
            fn()
        times = []
        t_start = time.perf_counter()
        while len(times) < min_runs:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if len(times) >= 3 and time.perf_counter() - t_start > budget_s:
                break
        times.sort()
        q = lambda f: times[min(len(times) - 1, int(f * len(times)))]  # noqa: E731
        return {"median_ms": round(statistics.median(times) * 1e3, 3), "p10_ms": round(q(0.1) * 1e3, 3),
                "p90_ms": round(q(0.9) * 1e3, 3), "runs": len(times)}

    legs = {"dequant_matmul": measure(dq_mm)}
    wf = [cpu_path.dequant(pk, sc).to(torch.float32) for pk, sc, _ in mats]
    legs["matmul_only"] = measure(mm)
    for leg in legs.values():
        t = leg["median_ms"] * 1e-3
        leg["GBps"] = round(nbytes / t / 1e9, 4)
        leg["GFLOPs"] = round(flops / t / 1e9, 2)
    return {"config": name, "bytes": nbytes, "flops": flops, "threads": torch.get_num_threads(), **legs}


def cpu_baseline(budget_s: float = 15.0):
    """The reference's CPU path (PyTorch restatement, oracle/cpu_path.py) on the host
    cores for the headline workload (configs[2], one 12B decode layer's linears at
    M=1): dequant + matmul per call, plus the matmul-only leg."""
    r = cpu_config("C3", budget_s)
    d, m = r["dequant_matmul"], r["matmul_only"]
    return {"value": d["GBps"], "unit": "GB/s", "cores": r["threads"], "kind": "port",
            "matmul_only": m["GBps"],
            "sample": f"one 12B decode layer's 6 W4A16 linears at M=1 (q,k,v,o,gate_up,down), torch CPU "
                      f"dequant+matmul per call (oracle/cpu_path.py): median {d['median_ms']} ms/step "
                      f"(p10 {d['p10_ms']}, p90 {d['p90_ms']}, {d['runs']} runs after 3 warm-ups); matmul only on "
                      f"pre-dequantized weights: median {m['median_ms']} ms/step ({m['GBps']} GB/s); "
                      f"threads {r['threads']} (affinity {len(os.sched_getaffinity(0))}, "
                      f"os.cpu_count() {os.cpu_count()}); cpu={cpu_model()}"}


def time_gate_up(torch, w4a16, o, M, K, F, unfused_leg=True):
    """Average duration of one fused w4a16_gate_up_gelu launch (h bf16 [M, F]) against the
    unfused composition (one linear over the concatenated [2F, K] weight, then torch's
    gelu(approximate="tanh") * mul on the bf16 halves), both as HIP graphs over weight sets
    larger than the MALL."""
    wbytes = 2 * (F * K // 2 + F * K // 16)
    nbytes = wbytes + 2 * M * K + 2 * M * F
    nsets = max(2, -(-ROTATE_BYTES // wbytes))
    sets = [make_set(torch, o, K, 2 * F, 7500 + i) for i in range(nsets)]
    lins = [(w4a16.W4Lin(pk[:F], sc[:F]), w4a16.W4Lin(pk[F:], sc[F:])) for pk, sc in sets]
    x = synth_x_dev(torch, o, M, K)
    h = torch.empty((M, F), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((M, 2 * F), dtype=torch.bfloat16, device="cuda")
    launches = nsets * max(1, -(-40 // nsets)) if M < 512 else nsets
    reps = 5 if M < 512 else 2

    def fused():
        for i in range(launches):
            g, u = lins[i % nsets]
            w4a16.gate_up_gelu(x, g, u, out=h)

    def unfused():
        for i in range(launches):
            pk, sc = sets[i % nsets]
            w4a16.linear(x, pk, sc, out=y)
            torch.mul(torch.nn.functional.gelu(y[:, :F], approximate="tanh"), y[:, F:], out=h)

    out = {"M": M, "K": K, "F": F, "bytes": nbytes, "flops": 4 * M * F * K, "sets": nsets, "launches": launches}
    legs = (("fused", fused), ("unfused", unfused)) if unfused_leg else (("fused", fused),)
    graphs = {name: graph_of(torch, fn) for name, fn in legs}
    for _ in range(2):  # alternate the legs and keep each one's best, so that order effects cancel
        for name, g in graphs.items():
            t = time_graph(torch, g, reps) / (reps * launches) * 1e6
            out[name + "_us"] = min(out.get(name + "_us", t), t)
    del graphs
    del sets, lins
    torch.cuda.empty_cache()
    t = out["fused_us"] * 1e-6
    out.update({"GBps": nbytes / t / 1e9, "TFLOPs": 4 * M * F * K / t / 1e12})
    return out


def time_lm_head(torch, w4a16, o, M, V, K, k):
    """Average duration of one w4a16_lm_head call (logits + softcap 30 + top-k) over one
    bf16 [V, K] embedding (2 GB at the 12B shape, larger than the MALL), as a HIP graph of
    back-to-back calls."""
    g = torch.Generator(device="cuda")
    g.manual_seed(9000)
    e = (torch.randn((V, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    x = synth_x_dev(torch, o, M, K)
    logits = torch.empty((M, V), dtype=torch.float32, device="cuda")
    ws = torch.empty(max(16, w4a16.lm_head_workspace_size(M, V, K, w4a16.DTYPE_BF16, k)), dtype=torch.uint8,
                     device="cuda")
    launches = 10

    def run():
        for _ in range(launches):
            w4a16.lm_head(x, e, softcap=30.0, topk=k, logits=logits, workspace=ws)

    gr = graph_of(torch, run)
    reps = 3
    t = time_graph(torch, gr, reps) / (reps * launches)
    del gr, e
    torch.cuda.empty_cache()
    nbytes = V * K * 2 + M * K * 2 + M * V * 4
    return {"M": M, "V": V, "K": K, "topk": k, "bytes": nbytes, "us": t * 1e6, "GBps": nbytes / t / 1e9,
            "hbm_frac": nbytes / t / 1e9 / PEAK_HBM_GBS}


def time_dequant(torch, w4a16, N, K):
    """Average durations of one w4a16_dequant call (bf16 [N, K] out) and one
    w4a16_unpack call (int8 [N, K] out), each a HIP graph of back-to-back calls
    rotating over packed weight sets larger than the MALL."""
    nsets = max(2, -(-ROTATE_BYTES // (N * K // 2 + N * K // 16)))
    sets = [make_set(torch, None, K, N, 7500 + i) for i in range(nsets)]
    w = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
    q = torch.empty((N, K), dtype=torch.int8, device="cuda")
    launches = nsets * max(1, -(-20 // nsets))
    out = {"N": N, "K": K, "launches": launches}
    for name, fn, nbytes in (
            ("dequant", lambda pk, sc: w4a16.dequantW4(pk, sc, out=w), N * K // 2 + N * K // 16 + 2 * N * K),
            ("unpack", lambda pk, sc: w4a16.unpackW4(pk, out=q), N * K // 2 + N * K)):
        def run(fn=fn):
            for i in range(launches):
                fn(*sets[i % nsets])
        g = graph_of(torch, run)
        t = time_graph(torch, g, 3) / (3 * launches)
        del g
        out[name] = {"bytes_per_call": nbytes, "avg_call_us": round(t * 1e6, 3), "GBps": round(nbytes / t / 1e9, 1),
                     "hbm_frac": round(nbytes / t / 1e9 / PEAK_HBM_GBS, 4)}
    del sets
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--all", action="store_true", help="also sweep every BASELINE config (stderr + gpurun_out)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--cpu-configs", action="store_true",
                    help="also time both CPU legs (dequant+matmul, matmul only) of every BASELINE config C1-C5")
    ap.add_argument("--only-dominant", action="store_true",
                    help="run only the dominant kernel's timing (gate_up, M=1): the workload of the committed "
                         "rocprofv3 kernel-trace and --pmc summaries")
    ap.add_argument("--config", type=str, default=None,
                    help="M,K,N: run only the timing of that one linear (graph of back-to-back launches over "
                         "weight sets larger than the MALL); the workload of the per-regime rocprofv3 summaries")
    ap.add_argument("--gate-up", type=str, default=None,
                    help="M,K,F: time only the fused gate/up + gelu*mul call (w4a16_gate_up_gelu) against the "
                         "unfused composition; the workload of the gate/up rocprofv3 summaries")
    ap.add_argument("--lm-head", type=str, default=None,
                    help="M,V,K,k: time only the lm_head call (logits, softcap 30, top-k); the workload of "
                         "its kernel traces")
    ap.add_argument("--dequant", type=str, default=None,
                    help="N,K: time only w4a16_dequant and w4a16_unpack on [N, K] weights; the workload of "
                         "their kernel traces")
    ap.add_argument("--no-unfused", action="store_true",
                    help="with --gate-up: time only the fused call (the workload of its kernel traces)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of known size (256 MiB read + 256 MiB write, 20 times): "
                         "the scale for rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the W4A16 linear would shard by rows of N; see DESIGN.md). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import torch
    import w4a16

    o = None  # the timed paths build their inputs with torch; only the CPU legs use oracle/
    w4a16.lib()  # fails loudly without the HIP library
    props = torch.cuda.get_device_properties(0)
    bi = build_info()
    log(f"BUILD: git={bi.get('git', '?')}{'-dirty' if bi.get('dirty') else ''} built={bi.get('built', '?')} "
        f"flags=\"{bi.get('flags', '?')}\" device={props.name} arch={getattr(props, 'gcnArchName', '?')} "
        f"CUs={props.multi_processor_count} clocks={gpu_clocks()} hip={torch.version.hip} torch={torch.__version__} "
        f"host={platform.node()}")

    if args.copy_calibration:
        n = 64 * 2**20
        src = torch.empty(n, dtype=torch.float32, device="cuda").uniform_()
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": {"read_bytes": 4 * n, "write_bytes": 4 * n, "launches": 20}}), flush=True)
        return 0

    if args.config:
        cM, cK, cN = (int(v) for v in args.config.split(","))
        r = time_config(torch, w4a16, o, cM, cK, cN)
        print(json.dumps({"M": cM, "K": cK, "N": cN, "bytes_per_launch": r["bytes"], "flops_per_launch": r["flops"],
                          "avg_launch_us": round(r["us"], 3), "GBps": round(r["GBps"], 1),
                          "TFLOPs": round(r["TFLOPs"], 2), "launches_per_replay": r["launches"]}), flush=True)
        return 0

    if args.gate_up:
        gM, gK, gF = (int(v) for v in args.gate_up.split(","))
        r = time_gate_up(torch, w4a16, o, gM, gK, gF, unfused_leg=not args.no_unfused)
        print(json.dumps({"M": gM, "K": gK, "F": gF, "bytes_per_launch": r["bytes"], "flops_per_launch": r["flops"],
                          "fused_us": round(r["fused_us"], 3),
                          "unfused_us": round(r["unfused_us"], 3) if "unfused_us" in r else None,
                          "GBps": round(r["GBps"], 1), "TFLOPs": round(r["TFLOPs"], 2),
                          "launches_per_replay": r["launches"]}), flush=True)
        return 0

    if args.dequant:
        qN, qK = (int(v) for v in args.dequant.split(","))
        print(json.dumps(time_dequant(torch, w4a16, qN, qK)), flush=True)
        return 0

    if args.lm_head:
        hM, hV, hK, hk = (int(v) for v in args.lm_head.split(","))
        r = time_lm_head(torch, w4a16, o, hM, hV, hK, hk)
        print(json.dumps({"M": hM, "V": hV, "K": hK, "topk": hk, "bytes_per_call": r["bytes"],
                          "avg_call_us": round(r["us"], 3), "GBps": round(r["GBps"], 1),
                          "hbm_frac": round(r["hbm_frac"], 4)}), flush=True)
        return 0

    if args.only_dominant:
        dom_name, dK, dN = [c for c in LAYER_12B if c[0] == DOMINANT][0]
        r = time_config(torch, w4a16, o, 1, dK, dN)
        print(json.dumps({"kernel": DOMINANT_KERNEL, "M": 1, "K": dK, "N": dN, "bytes_per_launch": r["bytes"],
                          "avg_launch_us": round(r["us"], 3), "GBps": round(r["GBps"], 1),
                          "launches_per_replay": r["launches"]}), flush=True)
        return 0

    # ---- the headline workload: 12B layer linears at M=1, rotating sets
    layer_bytes = sum(N * K // 2 + N * K // 16 for _, K, N in LAYER_12B)
    nsets = max(2, -(-ROTATE_BYTES // layer_bytes))
    log(f"allocating {nsets} weight sets of one 12B layer ({layer_bytes / 2**20:.1f} MiB each)")
    sets = [[make_set(torch, o, K, N, 1000 + 2 + 10 * s + i) for i, (_, K, N) in enumerate(LAYER_12B)]
            for s in range(nsets)]
    xs = {K: synth_x_dev(torch, o, 1, K) for K in {K for _, K, _ in LAYER_12B}}
    ys = [torch.empty((1, N), dtype=torch.bfloat16, device="cuda") for _, _, N in LAYER_12B]
    step_bytes = sum(lin_bytes(1, K, N) for _, K, N in LAYER_12B)
    dom = [i for i, (n, _, _) in enumerate(LAYER_12B) if n == DOMINANT][0]

    # q, k and v read the same x (engine.zig:552,571,583): one grouped call
    qkv = [i for i, (n, _, _) in enumerate(LAYER_12B) if n in ("q", "k", "v")]
    lins = [[w4a16.W4Lin(pk, sc) for pk, sc in ws] for ws in sets]

    def step(s):
        ws, ls = sets[s % nsets], lins[s % nsets]
        w4a16.linear_group(xs[LAYER_12B[qkv[0]][1]], [ls[i] for i in qkv], outs=[ys[i] for i in qkv])
        for i, (_, K, _) in enumerate(LAYER_12B):
            if i not in qkv:
                w4a16.linear(xs[K], ws[i][0], ws[i][1], out=ys[i])

    # eager (host-launched) steps, for reference: includes Python/ctypes launch overhead
    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / args.warmup * 1e3

    # timed region: one HIP graph per rotation of the weight sets (nsets steps),
    # replayed until `steps` steps have run, bracketed by synchronize + events
    g = graph_of(torch, lambda: [step(s) for s in range(nsets)])
    reps = max(1, -(-args.steps // nsets))
    steady(torch, g)
    # an event after every replay: the replay times give the step-time distribution
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record()
    for r in range(reps):
        g.replay()
        ev[r + 1].record()
    torch.cuda.synchronize()
    dt_wall = time.perf_counter() - t0
    n_steps = reps * nsets
    dt = ev[0].elapsed_time(ev[-1]) * 1e-3
    ms_per_step = dt / n_steps * 1e3
    value = step_bytes / (dt / n_steps) / 1e9
    per_step_us = sorted(ev[r].elapsed_time(ev[r + 1]) * 1e3 / nsets for r in range(reps))
    q = lambda f: per_step_us[min(len(per_step_us) - 1, int(f * len(per_step_us)))]  # noqa: E731
    dist = {"mean": round(dt / n_steps * 1e6, 3), "median": round(statistics.median(per_step_us), 3),
            "p10": round(q(0.1), 3), "p90": round(q(0.9), 3), "replays": reps, "steps_per_replay": nsets}
    del g

    # dominant kernel: graph of back-to-back gate_up launches over >= 8 weight sets
    dom_name, dK, dN = LAYER_12B[dom]
    dom = time_config(torch, w4a16, o, 1, dK, dN)
    dom_bytes, dom_avg, dom_gbs = dom["bytes"], dom["us"] * 1e-6, dom["GBps"]
    log(f"step us: median {dist['median']} p10 {dist['p10']} p90 {dist['p90']} over {reps} replays of {nsets} steps")
    log(f"step: {ms_per_step * 1e3:.2f} us ({value:.1f} GB/s, {value / PEAK_HBM_GBS * 100:.1f} % of HBM peak), "
        f"wall {dt_wall / n_steps * 1e6:.2f} us/step, eager {eager_ms * 1e3:.1f} us/step; "
        f"gate_up launch avg {dom_avg * 1e6:.2f} us = {dom_gbs:.1f} GB/s")
    del sets
    torch.cuda.empty_cache()

    # ---- M = 64: TFLOP/s of the 12B gate/up linear
    m64 = time_config(torch, w4a16, o, 64, 3840, 30720)
    log(f"M=64 gate_up: {m64['us']:.2f} us, {m64['TFLOPs']:.1f} TFLOP/s ({m64['mfma_frac'] * 100:.1f} % of bf16 MFMA), "
        f"{m64['GBps']:.0f} GB/s")

    table = None
    if args.all:
        table = []
        cfgs = [("C1", 1, 1536, 6144)]
        cfgs += [(f"E2B_{n}", 1, K, N) for n, K, N in [("q", 1536, 2048), ("kv", 1536, 256), ("o", 2048, 1536),
                                                        ("gate_up", 1536, 12288), ("down", 6144, 1536)]]
        cfgs += [(f"12B_{n}", 1, K, N) for n, K, N in LAYER_12B]
        # full-attention layers of the 12B (no v_proj): q 3840->8192, k 3840->512, o 8192->3840
        cfgs += [("12B_full_q", 1, 3840, 8192), ("12B_full_k", 1, 3840, 512), ("12B_full_o", 1, 8192, 3840)]
        # E2B per-layer-embedding linears (engine.zig:659, 661, 723)
        cfgs += [("E2B_ple_gate", 1, 1536, 256), ("E2B_ple_proj", 1, 256, 1536), ("E2B_plmp", 1, 1536, 8960)]
        # E2B double-wide MLP of the KV-shared layers 15-34: gate + up 1536->12288 each, down 12288->1536
        cfgs += [("E2B_dw_gate_up", 1, 1536, 24576), ("E2B_dw_down", 1, 12288, 1536)]
        cfgs += [(f"C4_M{M}", M, 3840, 30720) for M in (8, 16, 32, 64)]
        # configs[3] covers every config-2 weight at M = 8..64: the other linears of the layer
        cfgs += [(f"C4_{n}_M{M}", M, K, N) for M in (8, 16, 32, 64)
                 for n, K, N in LAYER_12B if n not in ("gate_up", "v")]
        cfgs += [("C5_gate_up", 2048, 3840, 30720), ("C5_down", 2048, 15360, 3840)]
        for name, M, K, N in cfgs:
            r = time_config(torch, w4a16, o, M, K, N)
            r["name"] = name
            table.append(r)
            log(f"{name:12s} M={M:5d} K={K:6d} N={N:6d}  {r['us']:9.2f} us"
                f"  {r['GBps']:8.1f} GB/s ({r['hbm_frac'] * 100:5.1f} %)  {r['TFLOPs']:8.2f} TFLOP/s ({r['mfma_frac'] * 100:5.1f} %)")
        # fused gate/up + gelu*mul (engine.zig:653) against the unfused composition
        for name, M, K, F in [("E2B_gelu", 1, 1536, 6144), ("E2B_dw_gelu", 1, 1536, 12288), ("12B_gelu", 1, 3840, 15360),
                              ("12B_gelu", 64, 3840, 15360), ("12B_gelu", 2048, 3840, 15360)]:
            r = time_gate_up(torch, w4a16, o, M, K, F)
            r["name"] = name
            table.append(r)
            log(f"{name:12s} M={M:5d} K={K:6d} F={F:6d}  fused {r['fused_us']:9.2f} us  unfused {r['unfused_us']:9.2f} us"
                f"  {r['GBps']:8.1f} GB/s  {r['TFLOPs']:8.2f} TFLOP/s")
        # w4a16_dequant / w4a16_unpack (W2/U1b shapes' largest matrices: 12B gate/up, down)
        for name, N, K in [("deq_12B_gate_up", 30720, 3840), ("deq_12B_down", 3840, 15360)]:
            r = time_dequant(torch, w4a16, N, K)
            r["name"] = name
            table.append(r)
            log(f"{name:15s} N={N:6d} K={K:6d}  dequant {r['dequant']['avg_call_us']:8.2f} us"
                f" ({r['dequant']['GBps']:7.1f} GB/s, {r['dequant']['hbm_frac'] * 100:4.1f} %)"
                f"  unpack {r['unpack']['avg_call_us']:8.2f} us ({r['unpack']['GBps']:7.1f} GB/s,"
                f" {r['unpack']['hbm_frac'] * 100:4.1f} %)")
        os.makedirs(os.path.join(ROOT, "gpurun_out"), exist_ok=True)
        with open(os.path.join(ROOT, "gpurun_out", "bench_all.json"), "w") as f:
            json.dump(table, f, indent=1)

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_budget)
    if cpu:
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['sample']})")
    cpu_table = None
    if (args.all or args.cpu_configs) and not args.no_cpu:
        cpu_table = []
        for name in CPU_CONFIGS:
            r = cpu_config(name, args.cpu_budget)
            cpu_table.append(r)
            d, m = r["dequant_matmul"], r["matmul_only"]
            log(f"cpu {name:7s} dequant+matmul {d['median_ms']:10.3f} ms ({d['GBps']:8.3f} GB/s, {d['GFLOPs']:8.2f} GFLOP/s)"
                f"  matmul only {m['median_ms']:10.3f} ms ({m['GBps']:8.3f} GB/s, {m['GFLOPs']:8.2f} GFLOP/s)"
                f"  threads {r['threads']}")
        os.makedirs(os.path.join(ROOT, "gpurun_out"), exist_ok=True)
        with open(os.path.join(ROOT, "gpurun_out", "cpu_configs.json"), "w") as f:
            json.dump(cpu_table, f, indent=1)

    traffic = read_traffic()
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (q ~ U{-8..7}, scale bf16(|N(0,1)|*0.02), x bf16 N(0,1); seeded)",
        "config": {"workload": "configs[2]: 12B-like decode layer linears at M=1 (q,k,v grouped in one call, o, "
                               "gate_up fused, down), bf16 x in / bf16 y out, int4 group 32",
                   "M": 1, "bytes_per_step": step_bytes, "weight_sets": nsets,
                   "hbm_frac": round(value / PEAK_HBM_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(dom_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "kernel": DOMINANT_KERNEL + " (12B gate_up, M=1, N=30720, K=3840)",
                     "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_avg * 1e6, 3)},
        "cpu_baseline": cpu,
        "m64": {"TFLOPs": round(m64["TFLOPs"], 2), "mfma_frac": round(m64["mfma_frac"], 4),
                "GBps": round(m64["GBps"], 1), "us": round(m64["us"], 2)},
        "timing": {"method": "HIP graph replays, events around the timed region and after every replay",
                   "step_us": dist, "eager_us_per_step": round(eager_ms * 1e3, 2)},
        "build": {"git": bi.get("git"), "dirty": bi.get("dirty"), "clocks": gpu_clocks()},
    }
    if cpu_table is not None:
        out["cpu_configs"] = cpu_table
    if table is not None:
        out["sweep"] = [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()} for r in table]
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
