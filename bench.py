"""Benchmark of the pjrtx hot path on one MI355X.

A step is one PJRT execute of the workload's compiled StableHLO program on
device-resident inputs (synthetic, seeded). Default workload: BASELINE
configs[1] — two-output max/index argmax over bf16 logits [64,128256] plus
f16 sum/max/min of the logits cast to f16 (one fused kernel). `--config c1`
runs configs[0] (f32 elementwise chain + row sum, [4096,4096]).

Prints one JSON line: whole-job HBM GB/s over algorithmic bytes, the
dominant kernel's roofline (HIP-event timed on the plugin's stream), and the
CPU oracle timed on this host as a reported baseline.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0

WORKLOADS = {
    "c2": dict(
        workload="argmax2_f16reduce_64x128256_bf16",
        desc="two-output argmax over logits [64,128256] bf16 + f16 sum/max/min of logits.astype(f16)",
        # read logits once + outputs (bf16 values, i32 indices, 3x f16)
        bytes=64 * 128256 * 2 + 64 * (2 + 4 + 3 * 2),
        # main pass reads every logit once; its partials stay in L2/MALL-sized scratch
        kernel_bytes=64 * 128256 * 2,
        dtype="bf16",
    ),
    "c1": dict(
        workload="f32_chain_rowsum_4096x4096",
        desc="sum(tanh(x*y+0.5)*x - max(y,0), axis=1), x,y [4096,4096] f32",
        bytes=2 * 4096 * 4096 * 4 + 4096 * 4,
        kernel_bytes=2 * 4096 * 4096 * 4 + 4096 * 4,
        dtype="f32",
    ),
    # Calibration only (not a bench line): a plain f32 stream of known size
    # whose FETCH_SIZE / WRITE_SIZE readings scale the other workloads' counters.
    "copy": dict(
        workload="stream_negate_8192x4096_f32",
        desc="out = -x, x [8192,4096] f32 (counter calibration)",
        bytes=2 * 8192 * 4096 * 4,
        kernel_bytes=2 * 8192 * 4096 * 4,
        dtype="f32",
    ),
}


def make(config: str):
    import numpy as np
    from oracle import ops  # input makers only; the timed path never calls the oracle
    from pjrtx_amd import programs
    if config == "c2":
        text = programs.c2_argmax_f16_reductions(64, 128256)
        inputs = [ops.c2_inputs(64, 128256, seed=0)]
        dtypes = ["bf16"]
    elif config == "copy":
        text = programs.stream_negate(8192, 4096)
        inputs = [np.random.default_rng(0).standard_normal((8192, 4096), dtype=np.float32)]
        dtypes = [None]
    else:
        text = programs.c1_elementwise_rowsum(4096, 4096)
        inputs = list(ops.c1_inputs(4096, 4096, seed=0))
        dtypes = [None, None]
    return text, inputs, dtypes


def cpu_baseline(config: str, inputs, budget_s: float = 10.0) -> dict:
    """The numpy oracle on this host's cores over the same workload, repeated
    for about `budget_s` seconds (a reported baseline, not the target)."""
    import numpy as np
    from oracle import ops
    fn = {"c2": lambda: ops.c2_reference(inputs[0]), "c1": lambda: ops.c1_rowsum(*inputs),
          "copy": lambda: np.negative(inputs[0])}[config]
    fn()
    n = 0
    t0 = time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s or n >= 1000:
            break
    per = el / n
    gbps = WORKLOADS[config]["bytes"] / per / 1e9
    return {"value": round(gbps, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"full workload x{n} calls of the numpy oracle ({per * 1e3:.1f} ms/call, single-threaded numpy)"}


def traffic_from_profiles(config: str):
    p = ROOT / "profiles" / f"{WORKLOADS[config]['workload']}_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            return None
    return None


def launch_units(plan: dict) -> list[dict]:
    """The plan's launch units in the order pjrtx_executable_time_steps
    reports them (a split reduction is a main and a combine unit), each with
    its algorithmic bytes (inputs read once + outputs written; 0 for a
    combine pass, which only reads the partial slots)."""
    units = []
    for st in plan["steps"]:
        if st["kind"] == "alias":
            units.append({"name": "-", "bytes": 0})
            continue
        name = st["name"] or ("lib:" + st.get("library", "?"))
        units.append({"name": name, "bytes": sum(st["in_bytes"]) + sum(st["out_bytes"])})
        if st["kind"] == "reduce" and st.get("splits", 1) > 1:
            units.append({"name": name + "_combine", "bytes": 0})
    return units


def bench_c5(a) -> int:
    """C5: greedy decode of the llama-like model. A step is one decode token
    (one PJRT execute of the decode program, caches donated). Prefill of the
    512-token prompt is timed separately and reported in `config`."""
    import numpy as np
    from pjrtx_amd import llama_like as L
    from pjrtx_amd.pjrt import Client
    cfg = L.FULL
    steps = min(a.steps, cfg.max_len - cfg.prompt)
    client = Client()
    t = time.perf_counter()
    weights = L.init_weights(cfg, seed=0)
    runner = L.LlamaRunner(client, cfg, weights)
    setup_s = time.perf_counter() - t
    prompt = L.prompt_tokens(cfg, seed=1)
    p = len(prompt)
    pos_bufs = [client.buffer(np.array(p + i, np.int32)) for i in range(steps)]

    tok, _, caches = runner.start(prompt)  # warmup: prefill + a few decode steps
    for i in range(min(a.warmup, steps)):
        tok, _, caches = runner.step_with(tok, pos_bufs[i], caches)
    tok.block_until_ready()

    t0 = time.perf_counter()
    tok, _, caches = runner.start(prompt)
    tok.block_until_ready()
    prefill_s = time.perf_counter() - t0
    toks = [tok]
    t0 = time.perf_counter()
    for i in range(steps):
        tok, _, caches = runner.step_with(tok, pos_bufs[i], caches)
        toks.append(tok)
    tok.block_until_ready()
    decode_s = time.perf_counter() - t0
    ms_per_step = decode_s * 1e3 / steps
    tokens = [int(x.to_numpy()[0]) for x in toks]

    # Per-launch timing of one decode step (HIP events on the plugin stream).
    plan = json.loads(runner.decode.optimized_program())
    units = launch_units(plan)
    args = runner.weights + [tok, pos_bufs[-1]] + caches
    unit_ms = runner.decode.time_steps(args, iters=20)
    names = runner.decode.step_names()
    assert len(units) == len(unit_ms) == len(names), (len(units), len(unit_ms), len(names))
    k = max(range(len(unit_ms)), key=lambda i: unit_ms[i] if units[i]["bytes"] else -1)
    kernel_ms = unit_ms[k]
    by_kind: dict[str, float] = {}
    for u, ms in zip(units, unit_ms):
        key = u["name"] if u["name"].startswith("lib:") else ("fusion_combine" if u["name"].endswith("_combine")
                                                               else "fusion")
        by_kind[key] = by_kind.get(key, 0.0) + ms * 1e3
    weight_bytes = 2 * L.num_params(cfg) - 2 * cfg.vocab * cfg.d_model + 2 * cfg.d_model  # one embedding row
    kv_bytes = 2 * cfg.layers * 2 * cfg.heads * cfg.head_dim * (cfg.max_len + 1)  # cache read over max_len + new row
    step_bytes = weight_bytes + kv_bytes
    line = {
        "metric": "llama-like decode tokens/s (greedy, batch 1)",
        "value": round(steps / decode_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights 0.02*N(0,1) seed 0, random 512-token prompt seed 1)",
        "config": {"workload": "llama_like_decode_8L_d2048_h16x128_ffn5632_v32000_prompt512",
                   "prefill_ms": round(prefill_s * 1e3, 3),
                   "prefill_tokens_per_s": round(p / prefill_s, 1),
                   "setup_s": round(setup_s, 1),
                   "decode_step_hbm_bytes": step_bytes,
                   "decode_step_gbps": round(step_bytes / (ms_per_step / 1e3) / 1e9, 1),
                   "launch_units_per_step": sum(1 for n in names if n != "-"),
                   "gpu_us_per_step_by_kind": {kk: round(v, 2) for kk, v in sorted(by_kind.items())},
                   "gpu_us_per_step": round(sum(unit_ms) * 1e3, 2),
                   "first_tokens": tokens[:8]},
        "roofline": {"bound": "hbm", "achieved": round(units[k]["bytes"] / (kernel_ms / 1e3) / 1e9, 2),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(units[k]["bytes"] / (kernel_ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": None, "kernel": names[k], "kernel_us": round(kernel_ms * 1e3, 3),
                     "kernel_algorithmic_bytes": units[k]["bytes"]},
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_c5(cfg, weights, prompt, tokens)
    print(json.dumps(line))
    return 0


def cpu_baseline_c5(cfg, weights, prompt, tokens, budget_s: float = 15.0) -> dict:
    """The numpy oracle decoding the same prompt (teacher-forced with the GPU's
    tokens) on this host, for about `budget_s` seconds of decode steps."""
    import numpy as np
    from oracle import llama as O
    W = O.weights_f32(cfg, weights)
    kc, vc = O.empty_caches(cfg)
    O.forward(cfg, W, prompt, 0, kc, vc)
    n, t0 = 0, time.perf_counter()
    while n < len(tokens) - 1:
        O.forward(cfg, W, np.array([tokens[n]], np.int32), len(prompt) + n, kc, vc)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    el = time.perf_counter() - t0
    import os
    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    return {"value": round(n / el, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} decode steps of the numpy oracle after the 512-token prefill "
                      f"({el / n * 1e3:.0f} ms/token, numpy matmul on all host cores)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", choices=sorted(WORKLOADS) + ["c5"], default="c2")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {a.gpus}); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        return 2

    if a.config == "c5":
        return bench_c5(a)

    from pjrtx_amd.pjrt import Client
    W = WORKLOADS[a.config]
    text, inputs, dtypes = make(a.config)
    client = Client()
    exe = client.compile(text)
    bufs = [client.buffer(x, dt) for x, dt in zip(inputs, dtypes)]
    for b in bufs:
        b.block_until_ready()

    for _ in range(a.warmup):
        outs = exe.execute_buffers(bufs)
    outs[-1].block_until_ready()
    del outs

    t0 = time.perf_counter()
    last = None
    for _ in range(a.steps):
        last = exe.execute_buffers(bufs)
    last[-1].block_until_ready()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / a.steps
    value = W["bytes"] / (ms_per_step / 1e3) / 1e9

    # Dominant kernel: per-launch HIP-event timing on the plugin's stream
    # (a split reduction's main and combine kernels are timed separately).
    unit_ms = exe.time_steps(bufs, iters=max(50, a.steps))
    names = exe.step_names()
    k = max(range(len(unit_ms)), key=lambda i: unit_ms[i])
    kernel_ms = unit_ms[k]
    achieved = W["kernel_bytes"] / (kernel_ms / 1e3) / 1e9

    line = {
        "metric": "fused-op HBM GB/s (% peak)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": W["dtype"],
        "data": "synthetic (seeded numpy inputs, resident in HBM before timing)",
        "config": {"workload": W["workload"], "desc": W["desc"], "algorithmic_bytes": W["bytes"],
                   "pct_hbm_peak_end_to_end": round(100 * value / HBM_PEAK_GBPS, 2),
                   "kernels_per_step": sum(1 for n in names if n != "-"),
                   "kernel_us": {n: round(t * 1e3, 3) for n, t in zip(names, unit_ms)}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic_from_profiles(a.config),
                     "kernel": names[k], "kernel_us": round(kernel_ms * 1e3, 3),
                     "kernel_algorithmic_bytes": W["kernel_bytes"]},
    }
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(a.config, inputs)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
