#!/usr/bin/env python3
"""Decode throughput of the gfx950 path on one MI355X, with the matvec
kernel's roofline fraction and the reference CPU path timed beside it.

Workload (default): TinyLlama-1.1B-shaped decoder, Q4 weights (Q8
activations), vocab 32000, synthetic N(0, 0.02) weights generated on the
device, a 64-token prompt and greedy decode with the KV cache growing to 320
positions.  A step is one greedy decode step (Model::logits with start_pos =
n - 1, device argmax, token fed back on the device), one replay of the
captured decode-step graph.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]

Prints one JSON line.  `value` is decode tokens/s over exactly K timed steps
(warmup steps run first, on the same sequence); `config.timed_positions`
gives the positions they cover.  `full_stream` times the workload's whole
greedy stream (every decode step after the prompt) and compares its tokens
with the reference's (tests/golden/<workload>.json).  `roofline` is for the
kernel that takes the most time in a decode step (the fused gate|up matvec
for the Q4/Q8 workloads): algorithmic bytes per launch (weights once + its
input rows + its output rows) over the launch's average duration, both
measured with HIP events recorded by the dispatches on the model stream,
during a second pass over the same timed steps with every kernel launched
directly; `per_kernel` gives the same figures for each matvec role.
`traffic` is the measured HBM bytes per launch of that kernel, from the
committed rocprofv3 counter summary (profiles/traffic.json), when one exists
for the workload and was taken on a build of the same kernel sources (the
summary records their digest); otherwise null, and `traffic_source` says
which build the committed counters belong to.

    python bench.py --copy-calibration MIB   (one plain copy of MIB MiB: the
                                              reference dispatch for the
                                              profiler's byte counters)
"""
import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "nanochatllms.cpp_amd")


def _load_package():
    if "nanochat_amd" in sys.modules:
        return sys.modules["nanochat_amd"]
    spec = importlib.util.spec_from_file_location("nanochat_amd", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["nanochat_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


nc = _load_package()

METRIC = "decode tok/s (1 GPU) + Q4/Q8 matvec HBM GB/s as % of MI355X peak"
HBM_PEAK_GBS = 8000.0
# kernel names (as the profiler lists them) of the fused decode matvecs
FUSED_KERNEL = {"qkv": "k_dmv_spec (q|k|v, residual add + norm prologue, weight terms beside the exact sums; "
                       "k_dmv where the speculative launch is not used)",
                "o": "k_dmv (o)",
                "gate_up": "k_dmv_glu_spec (gate|up, residual add + norm prologue beside the weight terms, "
                           "SwiGLU epilogue)",
                "down": "k_dmv (down)",
                "lm_head": "k_dmv_head (lm head in the head layout, residual add + final norm prologue, "
                           "greedy-token epilogue; k_dmv for widths other than 1280 / 1536 / 2048 / 2304)"}

FUSED_F16_KERNEL = {"qkv": "k_dmv_f16_nrm (q|k|v, residual add + norm prologue)",
                    "gate_up": "k_dmv_f16_nrm<GLU> (gate|up, residual add + norm prologue, SwiGLU epilogue)"}


def prompt_tokens(w):
    """The workload prompt (same generator as the tests), computed here
    without the checker: splitmix64 of (seed, stream, index) -> [0, vocab)."""
    mask = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        return z ^ (z >> 31)

    seed = w["seed"] + nc.PROMPT_SEED_OFFSET
    out = []
    for i in range(w["prompt"]):
        h = mix((seed * 0x9E3779B97F4A7C15 + 0x70CE5 * 0xD1B54A32D192ED03 + i) & mask)
        out.append(((h >> 32) * w["n_vocab"]) >> 32)
    return np.array(out, np.int32)


def host_info():
    """The host CPUs this process may run on: model name, logical CPUs,
    physical cores among them (distinct (package, core) pairs), their NUMA
    nodes, and the GPU's NUMA node when sysfs names it."""
    cpus = sorted(os.sched_getaffinity(0))
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cores, nodes = set(), set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}"
        try:
            with open(f"{base}/topology/physical_package_id") as f:
                pkg = f.read().strip()
            with open(f"{base}/topology/core_id") as f:
                core = f.read().strip()
            cores.add((pkg, core))
        except OSError:
            pass
        try:
            nodes.update(n[4:] for n in os.listdir(base) if n.startswith("node") and n[4:].isdigit())
        except OSError:
            pass
    gpu_node = None
    try:
        for card in sorted(os.listdir("/sys/class/drm")):
            p = f"/sys/class/drm/{card}/device/numa_node"
            if card.startswith("card") and "-" not in card and os.path.exists(p):
                with open(p) as f:
                    gpu_node = int(f.read().strip())
                break
    except (OSError, ValueError):
        pass
    return {"cpu_model": model, "logical_cpus": len(cpus), "physical_cores": len(cores) or None,
            "numa_nodes": sorted(int(n) for n in nodes), "gpu_numa_node": gpu_node,
            "affinity": f"{cpus[0]}-{cpus[-1]}" if cpus else None}


def cpu_baseline(w, prompt, budget_s=12.0):
    """The reference's own CPU path (oracle/_ref, built from its sources) on
    the same workload: untimed prefill, then greedy decode steps timed until
    the budget is spent.  Falls back to the oracle restatement ("port").
    The checker is loaded from tests/ for this leg only."""
    spec = importlib.util.spec_from_file_location("oracle_lib", os.path.join(ROOT, "tests", "oracle_lib.py"))
    OL = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(OL)
    kind = "reference" if OL.have_reference() else "port"
    lib = OL.Reference() if kind == "reference" else OL.Oracle()
    cfg = nc.workload_config(w["name"], cls=OL.Config)
    m = lib.model_create(cfg, w["seed"])
    toks = list(prompt)
    logits = np.zeros(cfg.n_vocab, np.float32)
    arr = np.array(toks, np.int32)
    lib.model_logits(m, OL.ptr(arr), len(arr), 0, OL.ptr(logits))
    toks.append(int(np.argmax(logits)))
    steps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s and len(toks) < cfg.max_ctx:
        arr = np.array(toks, np.int32)
        lib.model_logits(m, OL.ptr(arr), len(arr), len(arr) - 1, OL.ptr(logits))
        toks.append(int(np.argmax(logits)))
        steps += 1
    dt = time.perf_counter() - t0
    lib.model_free(m)
    hi = host_info()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or hi["logical_cpus"]
    return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": threads, "kind": kind,
            "sample": f"{steps} greedy decode steps after an untimed {len(prompt)}-token prefill "
                      f"({dt:.1f} s), same weights and prompt, OpenMP threads = {threads}",
            "host": hi}


def copy_calibration(mib):
    """One plain device copy of `mib` MiB (after a warmup copy): its counter
    readings under rocprofv3 --pmc scale the matvec kernels' FETCH_SIZE /
    WRITE_SIZE to bytes."""
    nc.init(0)
    n = mib << 20
    a, b = nc.DeviceBuffer(n), nc.DeviceBuffer(n)
    L = nc.lib()
    nc.check(L.nc_copy_d2d(C.c_void_p(b.ptr), C.c_void_p(a.ptr), n, None))
    nc.check(L.nc_synchronize())
    t0 = time.perf_counter()
    nc.check(L.nc_copy_d2d(C.c_void_p(b.ptr), C.c_void_p(a.ptr), n, None))
    nc.check(L.nc_synchronize())
    dt = time.perf_counter() - t0
    print(json.dumps({"copy_bytes": n, "copy_ms": round(dt * 1e3, 4)}), flush=True)


def kernel_sources_sha256(csrc_dir=os.path.join(PKG_DIR, "csrc")):
    """Digest of the library's sources (file names and contents, in name
    order): names the build a counter figure belongs to."""
    import hashlib
    h = hashlib.sha256()
    for name in sorted(os.listdir(csrc_dir)):
        path = os.path.join(csrc_dir, name)
        if os.path.isfile(path) and name.endswith((".hip", ".h", ".cpp")):
            h.update(name.encode() + b"\0")
            with open(path, "rb") as f:
                h.update(f.read())
            h.update(b"\0")
    return h.hexdigest()


def traffic_for(workload, kernel_role):
    """(HBM bytes per launch of the role's kernel from the committed counter
    summary or None, where that figure comes from).  The figure is given only
    when the summary was taken on a build of the same sources as this one."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None, "no counter summary"
    with open(path) as f:
        t = json.load(f)
    e = t.get(workload, {}).get(kernel_role)
    if e is None:
        return None, f"no counters for {workload} {kernel_role}"
    build = t.get("build", {})
    if build.get("kernel_sources_sha256") != kernel_sources_sha256():
        return None, (f"counters of build {build.get('commit', '?')} ({e['bytes_per_launch']} B per launch of "
                      f"{e['kernel']}); this build's kernel sources differ")
    return e["bytes_per_launch"], f"counters of this build ({build.get('commit', '?')})"


def reference_stream(workload):
    """The reference's greedy stream of the workload (golden fixture data)."""
    path = os.path.join(ROOT, "tests", "golden", f"{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)["tokens"]


def kernel_table(ms, nbytes, kind, wdtype):
    """Per matvec role: launches, total and average launch time, bytes per
    launch and the achieved rate."""
    out = []
    for k in sorted(set(kind.tolist())):
        sel = kind == k
        role = nc.PROF_ROLES[k & 7]
        fused = bool(k & nc.PROF_FUSED)
        avg_ms = float(ms[sel].mean())
        avg_b = float(nbytes[sel].mean())
        if wdtype == nc.F16:
            unfused = ("k_dmv_f16<GLU> (fp16 gate|up + SwiGLU decode matvec)" if role == "gate_up"
                       else "k_dmv_f16 (fp16 decode matvec)")
        else:
            unfused = "k_matvec_q"
        if fused and wdtype == nc.F16:
            kname = FUSED_F16_KERNEL[role]
        else:
            kname = FUSED_KERNEL[role] if fused else unfused
        out.append({"role": role, "kernel": kname,
                    "launches": int(sel.sum()), "total_ms": round(float(ms[sel].sum()), 4),
                    "avg_launch_us": round(avg_ms * 1e3, 3), "bytes_per_launch": round(avg_b),
                    "achieved_gbs": round(avg_b / (avg_ms * 1e-3) / 1e9, 1)})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=192)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--workload", default="tinyllama-q4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="launch every kernel directly instead of replaying "
                    "the captured decode-step graph (for profilers that do not follow graph launches)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB")
    ap.add_argument("--no-topk", action="store_true", help="skip the sampled-decode measurement")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); decode of these models runs as one "
              "independent stream per GPU, so N GPUs serve N streams at the 1-GPU rate.", file=sys.stderr)
        sys.exit(2)
    w = dict(nc.WORKLOADS[args.workload], name=args.workload)
    if args.warmup + args.steps > w["gen"] - 1:
        sys.exit(f"--warmup + --steps must be <= {w['gen'] - 1} for {args.workload}")

    if args.no_graph:
        os.environ["NC_DECODE_GRAPH"] = "0"
    nc.init(0)
    cfg = nc.workload_config(args.workload)
    model = nc.Model(cfg)
    model.init_synthetic(w["seed"])
    prompt = prompt_tokens(w)
    L = nc.lib()

    def sync():
        nc.check(L.nc_synchronize())

    # prefill (an untimed first one loads every kernel; the second is timed
    # on its own), warmup steps, then the timed steps (each step one replay
    # of the captured decode-step graph)
    model.prefill(prompt)
    sync()
    t0 = time.perf_counter()
    model.prefill(prompt)
    sync()
    prefill_s = time.perf_counter() - t0
    model.decode(args.warmup)
    sync()
    t0 = time.perf_counter()
    model.decode(args.steps)
    sync()
    dt = time.perf_counter() - t0
    timed_toks = model.decode(0, fetch=True)[: 1 + args.warmup + args.steps]
    # the whole stream: every decode step after the prompt, timed as one
    # call, its tokens compared with the reference's
    n_full = w["gen"] - 1
    model.prefill(prompt)
    sync()
    t0 = time.perf_counter()
    model.decode(n_full)
    sync()
    dt_full = time.perf_counter() - t0
    full_toks = model.decode(0, fetch=True)[: w["gen"]].tolist()
    ref = reference_stream(args.workload)
    full_stream = {"decode_tok_s": round(n_full / dt_full, 2), "steps": n_full,
                   "positions": [w["prompt"], w["prompt"] + n_full],
                   "matches_reference": None if ref is None else full_toks[: len(ref)] == ref,
                   "timed_tokens_match_reference": None if ref is None else
                   timed_toks.tolist() == ref[: len(timed_toks)]}
    # sampled decode (top-k 40, temperature 0.8, mt19937 seed 7): the same
    # step with the device sampler in place of the greedy pick; the rate is
    # the difference of two calls, prompt + first token and prompt + first
    # token + warmup + steps, after one call that captures the step graph
    topk_tok_s = None
    if not args.no_topk:
        topk_args = (0.8, 40, 7)
        model.generate_topk(prompt, 2, *topk_args)
        t0 = time.perf_counter()
        model.generate_topk(prompt, 1, *topk_args)
        t_one = time.perf_counter() - t0
        t0 = time.perf_counter()
        model.generate_topk(prompt, 1 + args.warmup + args.steps, *topk_args)
        t_all = time.perf_counter() - t0
        topk_tok_s = round((args.warmup + args.steps) / max(t_all - t_one, 1e-9), 2)
    # matvec timing: the same steps again (same positions, same tokens) with
    # direct launches, each matvec bracketed by HIP events on the model stream
    model.prefill(prompt)
    model.decode(args.warmup)
    launches_per_step = 4 * cfg.n_layers + 1
    model.profile_begin(launches_per_step * args.steps)
    t1 = time.perf_counter()
    model.decode(args.steps)
    sync()
    dt_direct = time.perf_counter() - t1
    model.profile_end()
    ms, nbytes, kind = model.profile_launches(launches_per_step * args.steps)
    model.close()

    per_kernel = kernel_table(ms, nbytes, kind, cfg.wdtype)
    dom = max(per_kernel, key=lambda e: e["total_ms"])
    traffic, traffic_source = traffic_for(args.workload, dom["role"])

    tok_s = args.steps / dt
    achieved = dom["achieved_gbs"]
    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if cfg.wdtype in (nc.Q4, nc.Q8) else "f16",
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: d_model {cfg.n_embd}, {cfg.n_layers} layers, "
                               f"{cfg.n_heads[0]}/{cfg.n_kv_heads[0]} heads, ffn {cfg.n_ffn[0]}, "
                               f"vocab {cfg.n_vocab}, prompt {w['prompt']}, greedy decode of "
                               f"{args.steps} timed steps after {args.warmup} warmup steps",
                   "prompt": w["prompt"], "max_ctx": cfg.max_ctx,
                   "timed_positions": [w["prompt"] + args.warmup, w["prompt"] + args.warmup + args.steps]},
        "full_stream": full_stream,
        "prefill_tok_s": round(w["prompt"] / prefill_s, 1),
        "direct_launch_tok_s": round(args.steps / dt_direct, 2),
        "topk_decode_tok_s": topk_tok_s,
        "topk_decode": "top_k 40, temperature 0.8, std::mt19937 seed 7; decode steps of one call (the graph "
                       "replays with the device sampler), prompt and first token subtracted",
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_source,
                     "kernel": dom["kernel"], "avg_launch_us": dom["avg_launch_us"],
                     "bytes_per_launch": dom["bytes_per_launch"], "launches": dom["launches"]},
        "per_kernel": per_kernel,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, prompt)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
