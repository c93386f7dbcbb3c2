"""Benchmark: ETHOS expert-layer forward tokens/s on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 20] [--config cfg2]
    python bench.py --config cfg5     # whole language-model forward (12 expert blocks)

A step is one full forward of the drop-in layer (query projection + BatchNorm,
product-key routing, reordering, expert generation, apply + scatter-back) over one
batch of synthetic input already resident in HBM.  Prints ONE JSON line.

Besides throughput, the line carries
  roofline      the dominant graded kernel (generator: MFMA, apply/scatter: HBM),
                algorithmic work per launch / mean launch time measured here with HIP
                events on the stream the kernels run on (every 4th timed step);
  kernels       the same figures for every stage;
  cpu_baseline  the reference's CPU path (a loop-faithful restatement of
                model.py:288-343, bit-identical to it on the golden fixtures) timed on a
                bounded token sample on this host, with every CPU the process may use;
  decode_64_tokens  the decode-like 64-token layer: p50 latency and its CPU baseline.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
FP32_PEAK_TFLOPS = 157.3     # MI355X fp32 (vector)
METRIC = "expert-layer fwd tokens/sec @1 MI355X; % HBM roofline + generator MFMA util"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def stage_work(sh, U: int) -> dict:
    """Algorithmic work per launch of each stage (bytes or flops)."""
    eb = 2 if sh.dtype == "bf16" else 4
    N = sh.n_pairs
    d, H, dq, K = sh.d_model, sh.num_heads, sh.d_query, sh.n_sub
    return {
        # x in, Wq in, q out
        "query_proj": dict(bound="hbm", work=(sh.n_tok * d + H * dq * d + sh.n_tok * H * dq) * eb, unit="GB/s"),
        # q in, both sub-key tables, gates + ids out
        "route": dict(bound="hbm", work=(sh.n_tok * H * dq + 2 * K * dq // 2) * eb + N * (eb + 4), unit="GB/s"),
        # 16 B per pair (key + value in and out) + slots
        "sort_segment": dict(bound="hbm", work=16 * N + 4 * (U + 1), unit="GB/s"),
        # 2 U (dl dh + dh d) flops: hidden rows and v rows of the unique experts
        "generate": dict(bound="mfma", work=2 * U * (sh.d_latent * sh.d_hidden + sh.d_hidden * d), unit="TFLOP/s"),
        # the per-unit bytes of the expert apply + scatter-back: u and v rows once per unique
        # expert (U 2d), x in and y out, expert id + gate + pair index per pair
        "apply_scatter": dict(bound="hbm", work=U * 2 * d * eb + 2 * sh.n_tok * d * eb + N * (4 + eb + 4),
                              unit="GB/s"),
    }


# Stage boundaries: three marked by the layer between its library calls, five recorded by
# the library inside the expert-stage call (ethos_stage_events).
OUTER = ["query_proj", "route", "sort_segment"]
INNER = ["token_proj", "hidden_rows", "activations", "v_rows", "scatter_back"]
# the graded stages as groups of those
STAGES = {"query_proj": ["query_proj"], "route": ["route"], "sort_segment": ["sort_segment"],
          "generate": ["hidden_rows", "v_rows"], "apply_scatter": ["token_proj", "activations", "scatter_back"]}


def timed_steps(m, x_flat, steps: int, every: int = 4) -> tuple[float, dict]:
    """Run `steps` layer forwards; return wall ms/step and the mean per-stage ms.

    Every step ends with one HIP event on the stream every kernel is launched on (torch's
    current stream, which the library is handed).  Steps 0, every, 2 every, ... also carry
    the stage boundaries, inside the same timed region: recorded by the layer between its
    calls, and by the library between the kernels of its expert-stage call.  A timed event
    between two kernels holds the GPU for a few microseconds (the nine of a step cost about
    27 us at 4096 tokens, 20 us at 64), so the other steps carry none; the per-stage means
    come from the instrumented steps, the p50 step time (`_p50`) from the others.
    """
    from ethos_amd import hip

    mk = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    det = list(range(0, steps, max(1, every)))
    bounds = [mk() for _ in range(steps + 1)]
    outer = {i: [mk() for _ in OUTER] for i in det}
    inner = {i: [mk() for _ in INNER] for i in det}
    for e in (ev for evs in inner.values() for ev in evs):
        e.record()  # the library records into existing events
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    bounds[0].record()
    for i in range(steps):
        if i in outer:
            pos = iter(outer[i])

            def mark(stage, pos=pos):
                next(pos).record()

            hip.stage_events(inner[i])
            try:
                m.forward_flat(x_flat, mark)
            finally:
                hip.stage_events([])  # the library holds no event past this step
        else:
            m.forward_flat(x_flat)
        bounds[i + 1].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    chain = {i: [bounds[i]] + outer[i] + inner[i] for i in det}
    per_k = {}
    for j, k in enumerate(OUTER + INNER):
        per_k[k] = sum(chain[i][j].elapsed_time(chain[i][j + 1]) for i in det) / len(det)
    per = {g: sum(per_k[k] for k in ks) for g, ks in STAGES.items()}
    per["_kernels"] = per_k
    plain = [i for i in range(steps) if i not in outer] or list(range(steps))
    steps_ms = sorted(bounds[i].elapsed_time(bounds[i + 1]) for i in plain)
    per["_p50"] = steps_ms[len(steps_ms) // 2]
    per["_instrumented"] = len(det)
    return elapsed / steps * 1e3, per


def hidden_rows_alone_ms(m, x_flat, reps: int = 20) -> float | None:
    """Mean time of the hidden-row kernel without its activation phase (ethos_generate with
    no v rows) on this batch's unique experts, timed with HIP events on the launch stream
    after the timed steps; None when the layer does not use the two-kernel generator."""
    from ethos_amd import hip

    if x_flat.dtype != torch.bfloat16:
        return None
    with torch.no_grad():
        _, ids = m.router.route(x_flat)
        seg = hip.sort_segment(ids.view(-1), m.num_experts)
        lat, w1, w2, _ = m._generator_params(x_flat.dtype, x_flat.device)
        run = lambda: hip.generate(lat, seg["uniq"], seg["n_unique"], seg["max_unique"], w1, w2,  # noqa: E731
                                   with_v=False)
        for _ in range(3):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def unique_experts(m, x_flat) -> int:
    from ethos_amd import hip

    with torch.no_grad():
        _, ids = m.router.route(x_flat)
        seg = hip.sort_segment(ids.view(-1), m.num_experts)
        return int(seg["n_unique"].item())


def load_profile_json(kind: str, config: str):
    """The machine-readable block of a committed rocprofv3 summary (profiles/<kind>_<config>.md),
    or None."""
    path = os.path.join(REPO, "profiles", f"{kind}_{config}.md")
    if not os.path.exists(path):
        return None
    try:
        return json.loads(open(path).read().split("```json", 1)[1].split("```", 1)[0])
    except (IndexError, ValueError):
        return None


def load_traffic(config: str, stage: str):
    """HBM bytes per launch of `stage` from the committed rocprofv3 --pmc summary (FETCH_SIZE +
    WRITE_SIZE, scaled by the same counters on a plain copy of known size), or None."""
    js = load_profile_json("hbm_traffic", config)
    try:
        return js["stages"][stage]["traffic_bytes"]
    except (TypeError, KeyError):
        return None


# Kernels behind the counter figures, named as rocprofv3 names them in the summaries.
SCATTER_KERNELS = ["void ethos::apply_scatter_kernel<u16, 2>"]
SORT_KERNELS = ["ethos::tsort_count", "void ethos::tsort_scan<false>", "void ethos::tsort_down<true>",
                "ethos::tsort_stats_map", "void ethos::tsort_scan<true>", "void ethos::tsort_down_last<false>",
                "ethos::tsort_pair_slot"]
GEMM_KERNELS = {"v_rows": "void ethos::expand_ws_bf16_kernel<512>",
                "hidden_rows_alone": "void ethos::hidden_ws_bf16_kernel<128, 512, false>",
                "hidden_rows_with_activations": "void ethos::hidden_ws_bf16_kernel<128, 512, true>"}


def counter_figures(config: str, stage_us: dict) -> dict | None:
    """Per-kernel evidence from the committed rocprofv3 counter summaries: HBM bytes per launch
    (FETCH_SIZE + WRITE_SIZE, copy-calibrated) of the gather/scatter and sort kernels over their
    launch time measured in this run, and the MFMA-busy fraction of the generator GEMMs
    (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs)."""
    hbm, mf = load_profile_json("hbm_traffic", config), load_profile_json("mfma_counters", config)
    out = {}
    if hbm and "kernels" in hbm:
        for stage, names in (("scatter_back", SCATTER_KERNELS), ("sort_segment", SORT_KERNELS)):
            ks = [k for k in names if k in hbm["kernels"]]
            us = stage_us.get(stage)
            if ks and us:
                b = sum(hbm["kernels"][k]["read_bytes"] + hbm["kernels"][k]["write_bytes"] for k in ks)
                gbs = b / (us * 1e-6) / 1e9
                out[stage] = dict(kernels=ks, hbm_bytes=b, us=us, achieved_GBps=round(gbs, 1), peak_GBps=HBM_PEAK_GBS,
                                  frac=round(gbs / HBM_PEAK_GBS, 4))
    if mf and "kernels" in mf:
        for name, k in GEMM_KERNELS.items():
            if k in mf["kernels"]:
                out[name] = dict(kernel=k, mfma_busy=mf["kernels"][k]["mfma_busy"])
    if not out:
        return None
    out["source"] = (f"profiles/hbm_traffic_{config}.md and profiles/mfma_counters_{config}.md (rocprofv3 counters); "
                     "times from this run")
    return out


def copy_probe(mib: int) -> None:
    """A plain device copy of `mib` MiB (read mib, write mib): the calibration kernel for the
    FETCH_SIZE / WRITE_SIZE counters."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    log(f"[bench] copy probe: neg over {mib} MiB fp32 ({n * 4} bytes read, {n * 4} bytes written) x3")
    del src, dst


def host_cpu() -> dict:
    """The host's CPU model (/proc/cpuinfo, else lscpu), its logical CPU count and the CPUs
    this process may run on."""
    model = None
    ident = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key == "model name" and model is None:
                    model = val.strip()
                elif key in ("cpu family", "model", "stepping") and key not in ident:
                    ident[key] = val.strip()
                if line.strip() == "":  # the first processor's block is enough
                    break
    except OSError:
        pass
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip() == "Model name" and val.strip() and (model is None or len(val.strip()) > len(model)):
                model = val.strip()
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    cpu_id = " ".join(f"{k} {ident[k]}" for k in ("cpu family", "model", "stepping") if k in ident)
    return {"cpu_model": model or "unknown", "cpu_id": cpu_id or "unknown", "logical_cpus": os.cpu_count(),
            "cpus_available": len(os.sched_getaffinity(0))}


def cpu_baseline(sh, x_cpu, sd_cpu, n_tokens: int) -> dict:
    from oracle import loop_faithful

    host = host_cpu()
    # every CPU this process may run on (the host's cores unless a CPU set restricts it)
    threads = host["cpus_available"]
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    xs = x_cpu[:n_tokens].contiguous()
    t0 = time.perf_counter()
    with torch.no_grad():
        loop_faithful.layer(xs, sd_cpu, sh.num_heads, sh.top_k)
    dt = time.perf_counter() - t0
    torch.set_num_threads(prev)
    # the vectorised oracle (numpy, float64 arithmetic with the reference's rounding points) on
    # the same sample, reported beside the loop-faithful port
    from oracle import oracle as O
    P = O.unpack_state(sd_cpu, sh.num_heads)
    n_vec = min(n_tokens, 64)  # its generator covers every unique expert of the sample: keep it short
    t1 = time.perf_counter()
    O.layer_forward(O.from_torch(xs[:n_vec]), P, sh.num_heads, sh.top_k, sh.dtype)
    dt_vec = time.perf_counter() - t1
    return {
        "value": round(n_tokens / dt, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": host["cpu_model"],
        "cpu_id": host["cpu_id"],
        "logical_cpus": host["logical_cpus"],
        "sample": f"first {n_tokens} of the {sh.n_tok} tokens of the same workload, full reference loop "
                  f"({n_tokens * sh.num_heads * sh.top_k} (token, head, k) iterations), {dt:.1f} s on "
                  f"{threads} threads",
        "vectorised_oracle": {"value": round(n_vec / dt_vec, 3), "unit": "tokens/s",
                              "sample": f"first {n_vec} tokens, {dt_vec:.1f} s"},
    }


def lm_forward(steps: int, warmup: int, alternatives: bool = True) -> dict:
    """Whole ETHOS LM forward (the reference's CompressedMoEModel with the drop-in expert
    layer in every block): 12 blocks, d_model 1024, MLA 16 heads with a 256-wide KV latent,
    vocabulary 100,277, batch 4 x 2048 uniform token ids, bf16, random init.  Returns ms per
    forward (HIP events around `steps` forwards), the expert layer's share (block 0's layer
    timed alone on its own input, times the block count) and, with `alternatives`, the same
    model with the expert layers in hidden-space order."""
    from ethos_amd.model import CompressedMoEModel, init_random_, lm_config
    cfg = lm_config()
    batch, seq = 4, 2048
    log("[bench] building the language model (random init on the host)")
    m = init_random_(CompressedMoEModel(cfg), seed=0).to(torch.bfloat16).cuda().eval()
    ids = torch.randint(0, cfg.vocab_size, (batch, seq), generator=torch.Generator().manual_seed(0)).cuda()
    out = {}
    with torch.no_grad():
        log("[bench] warmup")
        for _ in range(warmup):
            m(ids)
        torch.cuda.synchronize()
        log(f"[bench] timing {steps} model forwards")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            m(ids)
        e1.record()
        torch.cuda.synchronize()
        out["wall_ms"] = (time.perf_counter() - t0) / steps * 1e3
        out["ms"] = e0.elapsed_time(e1) / steps
        # one block's expert layer alone, on the block's actual input
        inputs = {}
        hk = m.layers[0].mlp.register_forward_pre_hook(lambda mod, a: inputs.__setitem__("x", a[0]))
        m(ids)
        hk.remove()
        x = inputs["x"]
        for _ in range(2):
            m.layers[0].mlp(x)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            m.layers[0].mlp(x)
        e1.record()
        torch.cuda.synchronize()
        out["ms_layer"] = e0.elapsed_time(e1) / steps
        if alternatives:
            # the same weights with the expert layers in hidden-space order
            for layer in m.layers:
                layer.mlp.hidden_space = True
            for _ in range(warmup):
                m(ids)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(steps):
                m(ids)
            e1.record()
            torch.cuda.synchronize()
            out["ms_hidden_space"] = e0.elapsed_time(e1) / steps
    out.update(cfg=cfg, batch=batch, seq=seq)
    del m
    torch.cuda.empty_cache()
    return out


def lm_workload(r: dict) -> str:
    cfg = r["cfg"]
    return (f"ETHOS LM forward, {cfg.num_layers} blocks (all expert layers), d_model {cfg.d_model}, MLA "
            f"{cfg.num_heads} heads kv {cfg.kv_lora_rank}, vocab {cfg.vocab_size}, tokens {r['batch']}x{r['seq']}, bf16")


def bench_model(args) -> None:
    """`--config cfg5`: the whole-model forward as the line's headline."""
    r = lm_forward(args.steps, args.warmup)
    cfg, ms = r["cfg"], r["ms"]
    n_tok = r["batch"] * r["seq"]
    line = {
        "metric": "ETHOS LM forward tokens/sec @1 MI355X",
        "value": round(n_tok / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "wall_ms_per_step": round(r["wall_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: uniform token ids, random-init weights",
        "config": {"workload": lm_workload(r), "num_layers": cfg.num_layers, "batch": r["batch"], "seq_len": r["seq"],
                   "parallelism": "single GPU"},
        "expert_layer_ms": round(r["ms_layer"], 4),
        "expert_layers_share": round(cfg.num_layers * r["ms_layer"] / ms, 4),
        "alternatives": {"hidden_space": dict(ms_per_step=round(r["ms_hidden_space"], 4),
                                              value=round(n_tok / (r["ms_hidden_space"] * 1e-3), 1),
                                              unit="tokens/s")},
    }
    print(json.dumps(line), flush=True)


def lm_block(steps: int, warmup: int) -> dict:
    """The whole-model forward for the default line: tokens/s, ms per forward and the share
    of the 12 expert layers (no hidden-space alternative, to keep the run short)."""
    r = lm_forward(steps, warmup, alternatives=False)
    cfg, ms = r["cfg"], r["ms"]
    n_tok = r["batch"] * r["seq"]
    return {"workload": lm_workload(r), "value": round(n_tok / (ms * 1e-3), 1), "unit": "tokens/s",
            "ms_per_forward": round(ms, 4), "steps": steps, "warmup": warmup,
            "expert_layer_ms": round(r["ms_layer"], 4),
            "expert_layers_share": round(cfg.num_layers * r["ms_layer"] / ms, 4)}


def skewed_block(steps: int, warmup: int) -> dict:
    """The large-batch skewed layer (32,768 tokens, sub-key rows scaled by (r+1)^-1.1, the
    262,144-expert layer, bf16): tokens/s over `steps` forwards, the p50 of the steps that
    carry no stage events, the stages' means and the unique-expert count."""
    import ethos_amd
    from ethos_amd.workloads import SHAPES, make_inputs

    sh = SHAPES["cfg4"]
    log(f"[bench] building inputs for {sh.name} ({sh.n_tok} tokens, skewed sub-keys)")
    x_cpu, sd_cpu = make_inputs(sh, seed=0)
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd_cpu)
    m = m.cuda().eval()
    x_flat = x_cpu.cuda().view(-1, sh.d_model)
    with torch.no_grad():
        for _ in range(warmup):
            m.forward_flat(x_flat)
        torch.cuda.synchronize()
        log(f"[bench] timing {steps} forwards of the {sh.n_tok}-token skewed layer")
        ms, st = timed_steps(m, x_flat, steps)
        U = unique_experts(m, x_flat)
    p50 = st.pop("_p50")
    st.pop("_instrumented")
    sub = st.pop("_kernels")
    del m
    torch.cuda.empty_cache()
    return {"workload": f"ETHOS expert-layer forward, {sh.n_tok} tokens x d_model {sh.d_model}, {sh.num_experts} "
                        f"experts, {sh.num_heads} routing heads, top-{sh.top_k}, Zipf(1.1)-skewed sub-keys, bf16",
            "value": round(sh.n_tok / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 4),
            "p50_step_ms": round(p50, 4), "steps": steps, "warmup": warmup, "unique_experts": U,
            "stage_us": {k: round(v * 1e3, 2) for k, v in sub.items()}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--cpu-tokens", type=int, default=1024, help="token sample for the CPU baseline (0 = skip)")
    ap.add_argument("--no-alternatives", action="store_true",
                    help="skip the hidden-space timing (profiling runs: keeps per-kernel averages to one order)")
    ap.add_argument("--no-decode", action="store_true", help="skip the 64-token layer's latency measurement")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the 32,768-token skewed layer and the whole-model forward blocks")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run a plain copy of this many MiB (counter calibration for profiling)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the expert layer is benchmarked at N=1 only "
              "(multi-GPU sharding is a design note, not part of this build)", file=sys.stderr)
        sys.exit(2)

    if args.config == "cfg5":
        bench_model(args)
        return

    import ethos_amd
    from ethos_amd.workloads import SHAPES, make_inputs

    sh = SHAPES[args.config]
    log(f"[bench] building inputs for {sh}")
    x_cpu, sd_cpu = make_inputs(sh, seed=0)
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd_cpu)
    m = m.cuda().eval()
    x = x_cpu.cuda().view(sh.batch, sh.n_tok // sh.batch, sh.d_model)

    if args.copy_probe_mib > 0:
        copy_probe(args.copy_probe_mib)
    x_flat = x.view(-1, sh.d_model)
    with torch.no_grad():
        log("[bench] warmup")
        for _ in range(args.warmup):
            m(x)
        torch.cuda.synchronize()
        log(f"[bench] timing {args.steps} steps")
        ms, st = timed_steps(m, x_flat, args.steps)
        p50 = st.pop("_p50")
        n_instr = st.pop("_instrumented")
        launch_ms = st.pop("_kernels")
        sub_us = {k: round(v * 1e3, 2) for k, v in launch_ms.items()}
        U = unique_experts(m, x_flat)
        # The hidden-row kernel also computes the activations of its tiles' pairs.  Its time is
        # split into the hidden rows (the same kernel without the activation phase, timed on
        # its own) and the activations (the rest, added to the activation kernel's).
        alone = hidden_rows_alone_ms(m, x_flat)
        split = None
        if alone is not None and launch_ms["hidden_rows"] > alone:
            act_part = launch_ms["hidden_rows"] - alone
            st["generate"] -= act_part
            st["apply_scatter"] += act_part
            split = {"hidden_rows_alone_us": round(alone * 1e3, 2), "activation_phase_us": round(act_part * 1e3, 2),
                     "note": "hidden_rows in stage_us is the kernel with its activation phase; generate counts "
                             "hidden_rows_alone_us, apply_scatter counts activation_phase_us"}
    work = stage_work(sh, U)
    kernels = {}
    for k, ms_k in st.items():
        w = work[k]
        if w["bound"] == "mfma":
            ach = w["work"] / (ms_k * 1e-3) / 1e12
            peak = BF16_PEAK_TFLOPS if sh.dtype == "bf16" else FP32_PEAK_TFLOPS
        else:
            ach = w["work"] / (ms_k * 1e-3) / 1e9
            peak = HBM_PEAK_GBS
        kernels[k] = dict(us=round(ms_k * 1e3, 2), bound=w["bound"], achieved=round(ach, 2), peak=peak,
                          unit=w["unit"], frac=round(ach / peak, 4), work=w["work"], parts=STAGES[k])
    # The generator as launched: the hidden-row kernel with its activation phase plus the
    # v-row kernel, next to the split figure graded above.
    if split is not None:
        raw_ms = launch_ms["hidden_rows"] + launch_ms["v_rows"]
        ach = work["generate"]["work"] / (raw_ms * 1e-3) / 1e12
        split["generate_in_pipeline"] = dict(us=round(raw_ms * 1e3, 2), achieved=round(ach, 2),
                                             peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                                             frac=round(ach / BF16_PEAK_TFLOPS, 4),
                                             note="hidden-row kernel with its activation phase + v-row kernel, "
                                                  "as launched in the timed steps")
    graded = {k: kernels[k] for k in ("generate", "apply_scatter")}
    dom = max(graded, key=lambda k: graded[k]["us"])
    kd = kernels[dom]
    roofline = dict(kernel=dom, bound=kd["bound"], achieved=kd["achieved"], peak=kd["peak"], unit=kd["unit"],
                    frac=kd["frac"], traffic=load_traffic(args.config, dom))

    # The paper's hidden-space reordering (Algorithm 1) of the same layer: no v rows, one
    # projection back per token.  Reported beside the headline, which measures the layer's
    # default execution order.
    alternatives = None
    if not args.no_alternatives:
        mh = ethos_amd.EthosExpertLayer(sh.config(), hidden_space=True).to(sh.torch_dtype)
        mh.load_state_dict(sd_cpu)
        mh = mh.cuda().eval()
        with torch.no_grad():
            for _ in range(args.warmup):
                mh(x)
            torch.cuda.synchronize()
            log(f"[bench] timing {args.steps} steps, hidden-space order")
            ms_h, st_h = timed_steps(mh, x_flat, args.steps)
            st_h.pop("_p50")
            st_h.pop("_kernels")
            st_h.pop("_instrumented")
        del mh
        alternatives = {"hidden_space": dict(
            ms_per_step=round(ms_h, 4), value=round(sh.n_tok / (ms_h * 1e-3), 1), unit="tokens/s",
            stage_us={k: round(v * 1e3, 2) for k, v in st_h.items()},
            note="paper Algorithm 1: h_acc = sum a h per token, one W_v projection; same function, "
                 "other rounding points (hidden_space=True)")}

    cpu = None
    if args.cpu_tokens > 0:
        log(f"[bench] CPU baseline on {args.cpu_tokens} tokens")
        cpu = cpu_baseline(sh, x_cpu, sd_cpu, args.cpu_tokens)

    decode = None
    if args.config == "cfg2" and not args.no_decode:
        decode = decode_latency(args, with_cpu=args.cpu_tokens > 0)
    skewed = lm = None
    if args.config == "cfg2" and not args.no_extra:
        del m
        torch.cuda.empty_cache()
        skewed = skewed_block(args.steps, max(args.warmup, 5))
        lm = lm_block(min(args.steps, 10), 3)

    line = {
        "metric": METRIC,
        "value": round(sh.n_tok / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "p50_step_ms": round(p50, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": sh.dtype,
        "data": "synthetic: seeded random inputs and random-init weights of the configured layer shape",
        "config": {
            "workload": f"ETHOS expert-layer forward, {sh.n_tok} tokens x d_model {sh.d_model}, "
                        f"{sh.num_experts} experts, {sh.num_heads} routing heads, top-{sh.top_k}, "
                        f"d_query {sh.d_query}, {sh.dtype}",
            "n_tok": sh.n_tok, "d_model": sh.d_model, "num_experts": sh.num_experts, "num_heads": sh.num_heads,
            "top_k": sh.top_k, "d_query": sh.d_query, "d_latent": sh.d_latent, "d_hidden": sh.d_hidden,
            "parallelism": "single GPU",
        },
        "unique_experts": U,
        "roofline": roofline,
        "kernels": kernels,
        "counters": counter_figures(args.config, sub_us),
        "stage_us": sub_us,
        "stage_events": f"stage boundaries recorded on {n_instr} of the {args.steps} timed steps "
                        "(every 4th, from the first); the others carry one event at their end",
        "hidden_rows_split": split,
        "alternatives": alternatives,
        "cpu_baseline": cpu,
        "decode_64_tokens": decode,
        "skewed_32768_tokens": skewed,
        "lm_forward": lm,
    }
    print(json.dumps(line), flush=True)


def captured_latency(m, x_flat, steps: int) -> dict:
    """The same forward replayed from a HIP graph (ethos_amd.graphs.CapturedLayer: one input
    copy and one graph launch per step): p50 of `steps` back-to-back steps, each bracketed by
    events, and whether the replay's output equals the eager forward's."""
    from ethos_amd.graphs import CapturedLayer

    cap = CapturedLayer(m, x_flat.shape[0])
    with torch.no_grad():
        same = bool(torch.equal(cap(x_flat), m.forward_flat(x_flat)))
        for _ in range(10):
            cap(x_flat)
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        ev[0].record()
        for i in range(steps):
            cap(x_flat)
            ev[i + 1].record()
        torch.cuda.synchronize()
    t = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
    p50 = t[len(t) // 2]
    return {"p50_ms": round(p50, 4), "value": round(x_flat.shape[0] / (p50 * 1e-3), 1),
            "unit": "tokens/s (at the p50 latency)", "steps": steps, "equals_eager": same,
            "note": "one input copy and one graph launch per step"}


def decode_latency(args, with_cpu: bool) -> dict:
    """The decode-like layer (64 tokens, the same 262,144-expert layer, bf16): p50 latency
    of the 40 of 50 forwards after warmup that carry no stage events (every 5th does), and
    the CPU port on all 64 tokens."""
    import ethos_amd
    from ethos_amd.workloads import SHAPES, make_inputs

    sh = SHAPES["cfg3"]
    x_cpu, sd_cpu = make_inputs(sh, seed=0)
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd_cpu)
    m = m.cuda().eval()
    x_flat = x_cpu.cuda()
    steps = 50
    with torch.no_grad():
        for _ in range(max(args.warmup, 5)):
            m.forward_flat(x_flat)
        torch.cuda.synchronize()
        log(f"[bench] timing {steps} forwards of the 64-token layer")
        ms, st = timed_steps(m, x_flat, steps, every=5)
    p50 = st.pop("_p50")
    st.pop("_kernels")
    st.pop("_instrumented")
    graph = captured_latency(m, x_flat, steps)
    out = {"workload": "ETHOS expert-layer forward, 64 tokens x d_model 1024, 262144 experts, 8 routing heads, "
                       "top-16, d_query 256, bf16",
           "p50_ms": round(p50, 4), "mean_ms": round(ms, 4), "steps": steps,
           "value": round(sh.n_tok / (p50 * 1e-3), 1), "unit": "tokens/s (at the p50 latency)",
           "stage_us": {k: round(v * 1e3, 2) for k, v in st.items()},
           "graph": graph}
    if with_cpu:
        log("[bench] CPU baseline on the 64-token layer")
        out["cpu_baseline"] = cpu_baseline(sh, x_cpu, sd_cpu, sh.n_tok)
    del m
    return out


if __name__ == "__main__":
    main()
