"""Benchmark: ETHOS expert-layer forward tokens/s on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--config cfg2]

A step is one full forward of the drop-in layer (query projection + BatchNorm,
product-key routing, reordering, expert generation, apply + scatter-back) over one
batch of synthetic input already resident in HBM.  Prints ONE JSON line.

Besides throughput, the line carries
  roofline      the dominant graded kernel (generator: MFMA, apply/scatter: HBM),
                algorithmic work per launch / mean launch time measured here with HIP
                events on the stream the kernels run on;
  kernels       the same figures for every stage;
  cpu_baseline  the reference's CPU path (a loop-faithful restatement of
                model.py:288-343, bit-identical to it on the golden fixtures) timed on a
                bounded token sample on this host.
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
        # 2 U (dl dh + dh 2d) flops
        "generate": dict(bound="mfma", work=2 * U * (sh.d_latent * sh.d_hidden + sh.d_hidden * 2 * d), unit="TFLOP/s"),
        # u and v once per unique expert, x in, y out, id + score + pair per pair
        "apply_scatter": dict(bound="hbm", work=U * 2 * d * eb + 2 * sh.n_tok * d * eb + N * (4 + eb + 4),
                              unit="GB/s"),
    }


def time_stages(m, x_flat, reps: int) -> tuple[dict, int]:
    """Mean per-stage time (ms) over `reps` forwards, HIP events on the current stream."""
    from ethos_amd import hip

    sh_names = ["query_proj", "route", "sort_segment", "generate", "apply_scatter"]
    acc = {k: 0.0 for k in sh_names}
    U = 0
    r = m.router
    for _ in range(reps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        wq, bq, k1, k2, alpha, beta = r._packed(x_flat.dtype, x_flat.device)
        lat, w1, w2 = m._generator_params(x_flat.dtype, x_flat.device)
        ev[0].record()
        q = hip.query_proj(x_flat, wq, bq, alpha, beta)
        ev[1].record()
        gates, ids = hip.route_topk(q, k1, k2, m.top_k)
        ev[2].record()
        seg = hip.sort_segment(ids.view(-1), m.num_experts)
        ev[3].record()
        uv = hip.generate(lat, seg["uniq"], seg["n_unique"], seg["max_unique"], w1, w2)
        ev[4].record()
        hip.apply_scatter(x_flat, uv, seg, gates, m.num_heads, m.top_k)
        ev[5].record()
        torch.cuda.synchronize()
        for i, k in enumerate(sh_names):
            acc[k] += ev[i].elapsed_time(ev[i + 1])
        U = int(seg["n_unique"].item())
    return {k: v / reps for k, v in acc.items()}, U


def cpu_baseline(sh, x_cpu, sd_cpu, n_tokens: int) -> dict:
    from oracle import loop_faithful

    threads = torch.get_num_threads()
    xs = x_cpu[:n_tokens].contiguous()
    t0 = time.perf_counter()
    with torch.no_grad():
        loop_faithful.layer(xs, sd_cpu, sh.num_heads, sh.top_k)
    dt = time.perf_counter() - t0
    return {
        "value": round(n_tokens / dt, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"first {n_tokens} of the {sh.n_tok} tokens of the same workload, full reference loop "
                  f"({n_tokens * sh.num_heads * sh.top_k} (token, head, k) iterations), {dt:.1f} s on "
                  f"{threads} threads",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg2")
    ap.add_argument("--cpu-tokens", type=int, default=96, help="token sample for the CPU baseline (0 = skip)")
    ap.add_argument("--stage-reps", type=int, default=10)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the expert layer is benchmarked at N=1 only "
              "(multi-GPU sharding is a design note, not part of this build)", file=sys.stderr)
        sys.exit(2)

    import ethos_amd
    from ethos_amd.workloads import SHAPES, make_inputs

    sh = SHAPES[args.config]
    log(f"[bench] building inputs for {sh}")
    x_cpu, sd_cpu = make_inputs(sh, seed=0)
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd_cpu)
    m = m.cuda().eval()
    x = x_cpu.cuda().view(sh.batch, sh.n_tok // sh.batch, sh.d_model)

    with torch.no_grad():
        log("[bench] warmup")
        for _ in range(args.warmup):
            m(x)
        torch.cuda.synchronize()
        log(f"[bench] timing {args.steps} steps")
        t0 = time.perf_counter()
        for _ in range(args.steps):
            m(x)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        log("[bench] per-stage timing")
        st, U = time_stages(m, x.view(-1, sh.d_model), args.stage_reps)

    ms = elapsed / args.steps * 1e3
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
                          unit=w["unit"], frac=round(ach / peak, 4), work=w["work"])
    graded = {k: kernels[k] for k in ("generate", "apply_scatter")}
    dom = max(graded, key=lambda k: graded[k]["us"])
    kd = kernels[dom]
    roofline = dict(kernel=dom, bound=kd["bound"], achieved=kd["achieved"], peak=kd["peak"], unit=kd["unit"],
                    frac=kd["frac"], traffic=None)

    cpu = None
    if args.cpu_tokens > 0:
        log(f"[bench] CPU baseline on {args.cpu_tokens} tokens")
        cpu = cpu_baseline(sh, x_cpu, sd_cpu, args.cpu_tokens)

    line = {
        "metric": METRIC,
        "value": round(sh.n_tok / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
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
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
