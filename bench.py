"""Benchmark of the pjrtx hot path on one MI355X.

A step is one PJRT execute of a workload's compiled StableHLO program on
device-resident inputs (synthetic, seeded). Workloads (`--config`), after
BASELINE.json's configs:

  c2       (configs[1]) two-output max/index argmax over bf16
           logits [64,128256] plus f16 sum/max/min of logits.astype(f16)
  c1       configs[0]: f32 elementwise chain + row sum, [4096,4096]
  c3mm     configs[2]: plain bf16 matmul [8192,8192] x [8192,8192]
  c3attn   configs[2]: attention dot_generals [8,32,2048,128], causal mask,
           f32 softmax, bf16 context
  c4g      configs[3]: embedding gather, table [128256,4096] bf16, idx [8,2048]
  c4s/c4i  configs[3]: Zipf(1.1) scatter-add of [1048576,256] updates into
           [65536,256], f32 / int32
  c5       configs[4]: llama-like greedy decode, tokens/s (a step is one token)
  topk     lax.top_k(logits, 50) over [64,128256] bf16 (sort row, not a
           BASELINE config)
  copy     counter calibration stream (not a bench line)

With no --config (the driver's run) the line's value is c2's, and the c5
decode (tokens/s, 128 greedy tokens) and c1 lines are measured in the same
process and carried in it as "c5" and "c1" objects.

Prints one JSON line: the whole-job rate, the dominant kernel's roofline
(HIP-event timed per launch on the plugin's stream) and, unless
--no-cpu-baseline, the numpy oracle timed on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time
from dataclasses import dataclass, field
from typing import Callable

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}


def host_threads() -> int:
    n = os.cpu_count() or 1
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


def host_facts() -> dict:
    """The host the CPU baseline ran on: logical CPUs, the CPUs this process
    may run on, the CPU model; and why the reference's own CPU figure (JAX's
    CPU backend) is not measured beside it."""
    model = None
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"os_cpu_count": os.cpu_count(), "affinity_cpus": affinity, "cpu_model": model,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "jax_cpu": "JAX CPU baseline unavailable: jax is not installed in this image and there is no network"}


def randn_bits(shape, seed: int, scale: float = 1.0):
    """Seeded N(0,1)*scale as bf16 bit patterns, filled in independently
    seeded 2^22-element blocks on a thread pool."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    out = np.empty(shape, np.uint16)
    flat = out.reshape(-1)

    def fill(blk):
        lo = blk << 22
        hi = min(flat.size, lo + (1 << 22))
        w = np.random.default_rng([seed, blk]).standard_normal(hi - lo, dtype=np.float32)
        w *= np.float32(scale)
        u = w.view(np.uint32)
        flat[lo:hi] = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    with ThreadPoolExecutor(min(16, host_threads())) as ex:
        list(ex.map(fill, range((flat.size + (1 << 22) - 1) >> 22)))
    return out


def randn_f32(shape, seed: int):
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    out = np.empty(shape, np.float32)
    flat = out.reshape(-1)

    def fill(blk):
        lo = blk << 22
        hi = min(flat.size, lo + (1 << 22))
        flat[lo:hi] = np.random.default_rng([seed, blk]).standard_normal(hi - lo, dtype=np.float32)

    with ThreadPoolExecutor(min(16, host_threads())) as ex:
        list(ex.map(fill, range((flat.size + (1 << 22) - 1) >> 22)))
    return out


def randint_s32(shape, seed: int, lo: int, hi: int):
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    out = np.empty(shape, np.int32)
    flat = out.reshape(-1)

    def fill(blk):
        lo_i = blk << 22
        hi_i = min(flat.size, lo_i + (1 << 22))
        flat[lo_i:hi_i] = np.random.default_rng([seed, blk]).integers(lo, hi, hi_i - lo_i, dtype=np.int32)

    with ThreadPoolExecutor(min(16, host_threads())) as ex:
        list(ex.map(fill, range((flat.size + (1 << 22) - 1) >> 22)))
    return out


@dataclass
class Workload:
    workload: str
    desc: str
    make: Callable        # () -> (program text, inputs, dtypes)
    bytes: int            # algorithmic HBM bytes per step
    dtype: str
    flops: int = 0        # per step (dot workloads)
    cpu: Callable | None = None  # (inputs) -> (callable, fraction of one step it does, sample text)
    meta: dict = field(default_factory=dict)


def _c1():
    from oracle import ops
    from pjrtx_amd import programs
    return programs.c1_elementwise_rowsum(4096, 4096), list(ops.c1_inputs(4096, 4096, seed=0)), [None, None]


def _c2():
    from oracle import ops
    from pjrtx_amd import programs
    return programs.c2_argmax_f16_reductions(64, 128256), [ops.c2_inputs(64, 128256, seed=0)], ["bf16"]


def _copy():
    from pjrtx_amd import programs
    return programs.stream_negate(8192, 4096), [randn_f32((8192, 4096), 0)], [None]


def _c3mm():
    from pjrtx_amd import programs
    s = 1.0 / 8192 ** 0.5
    return programs.c3_matmul(8192, 8192, 8192), [randn_bits((8192, 8192), 1, s), randn_bits((8192, 8192), 2, s)], \
        ["bf16", "bf16"]


def _c3attn():
    from pjrtx_amd import programs
    shp, s = (8, 32, 2048, 128), 1.0 / 128 ** 0.5
    return programs.c3_attention(*shp), [randn_bits(shp, 10 + i, s) for i in range(3)], ["bf16"] * 3


def _c4g():
    import numpy as np
    from pjrtx_amd import programs
    table = randn_bits((128256, 4096), 20, 0.02)
    idx = np.random.default_rng(21).integers(0, 128256, (8, 2048)).astype(np.int32)
    return programs.c4_embedding_gather(128256, 4096, 8, 2048), [table, idx], ["bf16", None]


def _c4s(dtype: str):
    import numpy as np
    from oracle import ops
    from pjrtx_amd import programs
    rows, dim, n = 65536, 256, 1048576
    idx = ops.zipf_indices(n, rows, seed=30)
    if dtype == "f32":
        x = np.zeros((rows, dim), np.float32)
        upd = randn_f32((n, dim), 31)
    else:
        x = np.zeros((rows, dim), np.int32)
        upd = randint_s32((n, dim), 31, -1000, 1000)
    return programs.c4_scatter_add(rows, dim, n, dtype), [x, idx, upd], [None, None, None]


def _topk():
    from oracle import ops
    from pjrtx_amd import programs
    return programs.topk_logits(64, 128256, 50), [ops.c2_inputs(64, 128256, seed=0)], ["bf16"]


# --------------------------------------------------------------- CPU legs

def _cpu_c1(inputs):
    from oracle import cbaseline
    t = cbaseline.host_threads()
    return ((lambda: cbaseline.c1(*inputs, threads=t)), 1.0,
            f"full workload, C restatement of the oracle (oracle/c/baseline.c, -O3 AVX2) on {t} host threads")


def _cpu_c2(inputs):
    from oracle import cbaseline
    t = cbaseline.host_threads()
    return ((lambda: cbaseline.c2(inputs[0], threads=t)), 1.0,
            f"full workload, C restatement of the oracle (oracle/c/baseline.c, -O3 AVX2) on {t} host threads")


def _cpu_copy(inputs):
    import numpy as np
    return (lambda: np.negative(inputs[0])), 1.0, "full workload, numpy negate"


def _cpu_c3mm(inputs):
    import numpy as np
    from oracle import ops
    a = ops.bf16_bits_to_f32(inputs[0][:1024])
    b = ops.bf16_bits_to_f32(inputs[1])
    return (lambda: np.matmul(a, b)), 1024 / 8192, "1024 of 8192 output rows, numpy f32 matmul (BLAS, all host threads)"


def _cpu_c3attn(inputs):
    from oracle import ops
    q, k, v = (t[0, :2] for t in inputs)
    return (lambda: ops.attention_bf16(q, k, v)), 2 / 256, "2 of 256 (batch, head) pairs, numpy oracle"


def _cpu_c4g(inputs):
    from oracle import ops
    return (lambda: ops.gather_rows(inputs[0], inputs[1])), 1.0, "full workload, numpy gather"


def _cpu_c4s(inputs):
    from oracle import ops
    x, idx, upd = inputs
    n = len(idx) // 64
    fn = ops.scatter_rows_add if x.dtype.kind == "f" else ops.scatter_rows_add_int
    return (lambda: fn(x, idx[:n], upd[:n])), 1 / 64, "1/64 of the updates, numpy np.add.at in update order"


def _cpu_topk(inputs):
    from oracle import sort
    return (lambda: sort.top_k(inputs[0], 50, bf16=True)), 1.0, "full workload, numpy oracle (stable argsort)"


WORKLOADS = {
    "c2": Workload("argmax2_f16reduce_64x128256_bf16",
                   "two-output argmax over logits [64,128256] bf16 + f16 sum/max/min of logits.astype(f16)",
                   _c2, 64 * 128256 * 2 + 64 * (2 + 4 + 3 * 2), "bf16", cpu=_cpu_c2),
    "c1": Workload("f32_chain_rowsum_4096x4096", "sum(tanh(x*y+0.5)*x - max(y,0), axis=1), x,y [4096,4096] f32",
                   _c1, 2 * 4096 * 4096 * 4 + 4096 * 4, "f32", cpu=_cpu_c1),
    "c3mm": Workload("bf16_matmul_8192x8192x8192", "bf16 [8192,8192] x [8192,8192] -> bf16, f32 accumulation",
                     _c3mm, 3 * 8192 * 8192 * 2, "bf16", flops=2 * 8192 ** 3, cpu=_cpu_c3mm),
    "c3attn": Workload("attention_8x32x2048x128_causal_bf16",
                       "scores=einsum(bhqd,bhkd), causal select, f32 softmax, context=einsum(bhqk,bhkd) -> bf16",
                       _c3attn, 2 * 2415919104 + 4294967296, "bf16", flops=2 * 274877906944, cpu=_cpu_c3attn),
    "c4g": Workload("embedding_gather_128256x4096_bf16_idx8x2048", "table[idx], table [128256,4096] bf16",
                    _c4g, 16384 * 4096 * 2 + 65536 + 16384 * 4096 * 2, "bf16", cpu=_cpu_c4g),
    "c4s": Workload("scatter_add_zipf1.1_1048576x256_into_65536_f32",
                    "operand.at[idx].add(updates), Zipf(1.1) idx, f32, deterministic update order",
                    lambda: _c4s("f32"), 1073741824 + 4194304 + 2 * 67108864, "f32", cpu=_cpu_c4s),
    "c4i": Workload("scatter_add_zipf1.1_1048576x256_into_65536_s32",
                    "operand.at[idx].add(updates), Zipf(1.1) idx, int32 (bit-exact)",
                    lambda: _c4s("s32"), 1073741824 + 4194304 + 2 * 67108864, "int32", cpu=_cpu_c4s),
    "topk": Workload("top_k50_64x128256_bf16", "lax.top_k(logits, 50), logits [64,128256] bf16 (chlo.top_k)",
                     _topk, 64 * 128256 * 2 + 64 * 50 * (2 + 4), "bf16", cpu=_cpu_topk),
    # Calibration only (not a bench line): a plain f32 stream of known size
    # whose FETCH_SIZE / WRITE_SIZE readings scale the other workloads' counters.
    "copy": Workload("stream_negate_8192x4096_f32", "out = -x, x [8192,4096] f32 (counter calibration)",
                     _copy, 2 * 8192 * 4096 * 4, "f32", cpu=_cpu_copy),
}


def cpu_baseline(W: Workload, inputs, budget_s: float = 10.0) -> dict:
    """The numpy oracle on this host over a bounded sample of the workload,
    repeated for about `budget_s` seconds (a reported baseline, not the
    target), scaled to the full step."""
    fn, frac, sample = W.cpu(inputs)
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s or n >= 100000:
            break
    step_s = el / n / frac
    out = {"unit": "TFLOP/s" if W.flops else "GB/s", "cores": host_threads(), "kind": "port",
           "sample": f"{sample}; {n} calls, {el / n * 1e3:.1f} ms/call"}
    out["value"] = round(W.flops / step_s / 1e12, 4) if W.flops else round(W.bytes / step_s / 1e9, 3)
    if "BLAS" not in sample and "host threads" not in sample:
        out["cores"] = 1  # numpy elementwise / indexing runs on one thread
    out["host"] = host_facts()
    return out


def launch_units(plan: dict) -> list[dict]:
    """The plan's launch units in the order pjrtx_executable_time_steps
    reports them (a split reduction with a separate combine kernel is a main
    and a combine unit), each with
    its algorithmic bytes (the planner's figure: inputs read once + outputs
    written, gathered rows only for a gather, the window only for an in-place
    dynamic_update_slice; 0 for a combine pass, which only reads the partial
    slots) and dot flops."""
    units = []
    for st in plan["steps"]:
        if st["kind"] == "alias":
            units.append({"name": "-", "bytes": 0, "flops": 0})
            continue
        name = st["name"] or ("lib:" + st.get("library", "?"))
        # A causal attention step does (and is credited with) only the
        # unmasked (query, key) pairs.
        units.append({"name": name, "bytes": st["algorithmic_bytes"],
                      "flops": st.get("effective_flops", st.get("flops", 0))})
        if st["kind"] == "reduce" and st.get("splits", 1) > 1 and not st.get("fused_combine", False):
            units.append({"name": name + "_combine", "bytes": 0, "flops": 0})
    return units


def profile_unit_us(workload: str, unit: str):
    """The rocprofv3 figure for `unit` that the committed kernel-stats summary
    of this workload records (its `rocprof_unit_us <unit> <us> [route]` line:
    the unit's kernels' total duration over the run divided by the unit's
    calls), so that `frac` can be recomputed from the profile. A plain GEMM
    has two routes (the own kernels, or hipBLASLt with PJRTX_BLASLT=1),
    each with its own summary."""
    route = "blaslt" if os.environ.get("PJRTX_BLASLT", "0") == "1" else "own"
    for p in sorted((ROOT / "profiles").glob(f"*.{workload}.kernel_stats.md")):
        for ln in p.read_text().splitlines():
            parts = ln.strip().strip("`").split()
            if len(parts) >= 3 and parts[0] == "rocprof_unit_us" and parts[1] == unit:
                if len(parts) >= 4 and parts[3] != route:
                    continue
                return {"file": f"profiles/{p.name}", "kernel_us": float(parts[2])}
    return None


_MEASURED_PEAK = {}


def measured_mfma_peak() -> float | None:
    """Dense bf16 MFMA TFLOP/s this GPU sustains (pjrtx_mfma_peak_tflops,
    v_mfma_f32_32x32x16_bf16 on every SIMD), measured once per process."""
    if "bf16" not in _MEASURED_PEAK:
        from pjrtx_amd.pjrt import plugin
        try:
            _MEASURED_PEAK["bf16"] = round(max(plugin().mfma_peak_tflops(0, 1) for _ in range(2)), 1)
        except Exception:
            _MEASURED_PEAK["bf16"] = None
    return _MEASURED_PEAK["bf16"]


def roofline(units, unit_ms, names, dtype: str, workload: str | None = None) -> dict:
    """Roofline of the dominant launch unit: HBM-bound unless its arithmetic
    intensity is past the MFMA ridge point. `kernel_us` is the HIP-event time
    of the unit replayed back to back on the plugin's stream; `rocprof` is the
    committed profile's figure for the same unit, with the fraction it gives."""
    k = max(range(len(unit_ms)), key=lambda i: unit_ms[i] if units[i]["bytes"] else -1)
    u, sec = units[k], unit_ms[k] / 1e3
    peak_tf = MFMA_PEAK_TFLOPS.get(dtype, MFMA_PEAK_TFLOPS["bf16"])
    ridge = peak_tf * 1e12 / (HBM_PEAK_GBPS * 1e9)
    out = {"kernel": names[k], "kernel_us": round(unit_ms[k] * 1e3, 3), "kernel_algorithmic_bytes": u["bytes"]}
    prof = profile_unit_us(workload, names[k]) if workload else None
    if u["flops"] and u["flops"] / max(u["bytes"], 1) > ridge:
        ach = u["flops"] / sec / 1e12
        out.update({"bound": "mfma", "achieved": round(ach, 2), "peak": peak_tf, "unit": "TFLOP/s",
                    "frac": round(ach / peak_tf, 4), "kernel_flops": u["flops"]})
        mp = measured_mfma_peak() if dtype in ("bf16", "f16") else None
        if mp:
            out["measured_peak"] = mp
            out["frac_of_measured_peak"] = round(ach / mp, 4)
        if prof:
            prof["frac"] = round(u["flops"] / (prof["kernel_us"] * 1e-6) / 1e12 / peak_tf, 4)
    else:
        ach = u["bytes"] / sec / 1e9
        out.update({"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(ach / HBM_PEAK_GBPS, 4)})
        if u["flops"]:
            out["kernel_tflops"] = round(u["flops"] / sec / 1e12, 2)
        if prof:
            prof["frac"] = round(u["bytes"] / (prof["kernel_us"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)
    if prof:
        out["rocprof"] = prof
    keys = ["bound", "achieved", "peak", "unit", "frac"]
    return {**{kk: out[kk] for kk in keys}, "traffic": None, **{kk: v for kk, v in out.items() if kk not in keys}}


def unit_table(names, unit_ms) -> dict:
    """Per-launch-unit microseconds; repeated names get a #k suffix."""
    out, seen = {}, {}
    for n, t in zip(names, unit_ms):
        if n == "-":
            continue
        k = seen.get(n, 0)
        seen[n] = k + 1
        out[n if k == 0 else f"{n}#{k}"] = round(t * 1e3, 3)
    return out


def traffic_from_profiles(workload: str, kernel: str):
    """HBM bytes per launch of `kernel`, from the counter summary committed
    under profiles/ (null when that kernel was not profiled). A plain GEMM on
    the hipBLASLt route (PJRTX_BLASLT=1) reads its own summary."""
    names = [f"{workload}_traffic.json"]
    if os.environ.get("PJRTX_BLASLT", "0") == "1":
        names.insert(0, f"{workload}_blaslt_traffic.json")
    for name in names:
        p = ROOT / "profiles" / name
        if not p.exists():
            continue
        try:
            d = json.loads(p.read_text())
        except Exception:
            return None
        if d.get("kernel") == kernel:
            return d.get("hbm_bytes_per_launch")
    return None


def bench_program(a, W: Workload) -> dict:
    from pjrtx_amd.pjrt import Client
    text, inputs, dtypes = W.make()
    client = Client()
    exe = client.compile(text)
    bufs = [client.buffer(x, dt) for x, dt in zip(inputs, dtypes)]
    for b in bufs:
        b.block_until_ready()
    outs = None
    for _ in range(a.warmup):
        outs = exe.execute_buffers(bufs)
    if outs:
        outs[-1].block_until_ready()
    del outs
    # The timed region is the plugin's own execute loop (pjrtx_executable_run:
    # the PJRT execute path, synchronized before and after), so the ctypes
    # client's per-call cost is left out; the Python-loop figure is reported
    # beside it.
    ms_per_step = exe.run_loop(bufs, a.steps) / a.steps
    # The same loop through the PJRT C API (one PJRT_LoadedExecutable_Execute
    # per step, its event and outputs destroyed), beside it.
    pjrt_ms_per_step = exe.run_loop_pjrt(bufs, a.steps) / a.steps
    t0 = time.perf_counter()
    last = None
    for _ in range(a.steps):
        last = exe.execute_buffers(bufs)
    last[-1].block_until_ready()
    py_ms_per_step = (time.perf_counter() - t0) * 1e3 / a.steps
    del last

    plan = json.loads(exe.optimized_program())
    units = launch_units(plan)
    unit_ms = exe.time_steps(bufs, iters=max(10, min(50, a.steps)))
    names = exe.step_names()
    assert len(units) == len(unit_ms) == len(names), (len(units), len(unit_ms), len(names))
    rf = roofline(units, unit_ms, names, W.dtype, W.workload)
    rf["traffic"] = traffic_from_profiles(W.workload, rf["kernel"])
    sec = ms_per_step / 1e3
    if W.flops:
        metric, value, unit = "dot_general TFLOP/s (% MFMA peak)", W.flops / sec / 1e12, "TFLOP/s"
        pct = 100 * value / MFMA_PEAK_TFLOPS.get(W.dtype, 2500.0)
    else:
        metric, value, unit = "fused-op HBM GB/s (% peak)", W.bytes / sec / 1e9, "GB/s"
        pct = 100 * value / HBM_PEAK_GBPS
    line = {
        "metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": W.dtype,
        "data": "synthetic (seeded numpy inputs, resident in HBM before timing)",
        "config": {"workload": W.workload, "desc": W.desc, "algorithmic_bytes": W.bytes,
                   **({"flops": W.flops} if W.flops else {}),
                   "pct_peak_end_to_end": round(pct, 2),
                   "hbm_gbps_end_to_end": round(W.bytes / sec / 1e9, 2),
                   "kernels_per_step": sum(1 for n in names if n != "-"),
                   "pjrt_c_api_ms_per_step": round(pjrt_ms_per_step, 5),
                   "python_client_ms_per_step": round(py_ms_per_step, 5),
                   "kernel_us": unit_table(names, unit_ms)},
        "roofline": rf,
    }
    if not a.no_cpu_baseline and W.cpu:
        line["cpu_baseline"] = cpu_baseline(W, inputs)
    return line


def bench_c5(a, extras: bool = True) -> dict:
    """C5: greedy decode of the llama-like model. A step is one decode token
    (one PJRT execute of the decode program, caches donated). Prefill of the
    512-token prompt is timed separately and reported in `config`. `extras`
    adds the forced-graph and one-execute (on-device loop) rates beside the
    per-token one."""
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
    # Weight upload rate (pageable numpy -> HBM, the staged H2D path).
    t = time.perf_counter()
    again = [client.buffer(w, "bf16") for w in weights]
    for wb in again:
        wb.block_until_ready()
    upload_s = time.perf_counter() - t
    upload_bytes = sum(w.nbytes for w in weights)
    del again
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

    graph_stats = runner.decode.graph_stats()
    # The same decode loop with every execute replayed as a hipGraph
    # (PJRTX_GRAPHS=2), for comparison: the default captures only launch-bound
    # plans, and this one runs eagerly. Skipped when the caller set
    # PJRTX_GRAPHS (profiling runs keep graphs off).
    graph_ms = None
    if extras and "PJRTX_GRAPHS" not in os.environ:
        os.environ["PJRTX_GRAPHS"] = "2"
        try:
            tok_e, _, caches_e = runner.start(prompt)
            for i in range(min(3, steps)):
                tok_e, _, caches_e = runner.step_with(tok_e, pos_bufs[i], caches_e)
            tok_e, _, caches_e = runner.start(prompt)
            tok_e.block_until_ready()
            t0 = time.perf_counter()
            for i in range(steps):
                tok_e, _, caches_e = runner.step_with(tok_e, pos_bufs[i], caches_e)
            tok_e.block_until_ready()
            graph_ms = round((time.perf_counter() - t0) * 1e3 / steps, 4)
            del caches_e
        finally:
            os.environ.pop("PJRTX_GRAPHS")

    # All decode steps in one execute: the step inside an on-device while
    # loop over a constant count (compiled and warmed before timing).
    loop_ms, loop_match = None, None
    if extras:
        looped = client.compile(L.generate_program(cfg, steps))
        tok_l, _, caches_l = runner.start(prompt)
        looped.execute_buffers(runner.weights + [tok_l, pos_bufs[0]] + caches_l)[0].block_until_ready()
        tok_l, _, caches_l = runner.start(prompt)
        tok_l.block_until_ready()
        t0 = time.perf_counter()
        outs_l = looped.execute_buffers(runner.weights + [tok_l, pos_bufs[0]] + caches_l)
        outs_l[0].block_until_ready()
        loop_ms = round((time.perf_counter() - t0) * 1e3 / steps, 4)
        loop_match = [int(x) for x in outs_l[0].to_numpy()] == tokens[1:]
        del outs_l, caches_l

    plan = json.loads(runner.decode.optimized_program())
    units = launch_units(plan)
    args = runner.weights + [tok, pos_bufs[-1]] + caches
    unit_ms = runner.decode.time_steps(args, iters=20)
    names = runner.decode.step_names()
    assert len(units) == len(unit_ms) == len(names), (len(units), len(unit_ms), len(names))
    by_kind: dict[str, float] = {}
    for u, ms in zip(units, unit_ms):
        n = u["name"]
        key = (n if n.startswith("lib:") else "gemv" if n.startswith("pjrtx_gemv") else
               "fusion_combine" if n.endswith("_combine") else "fusion")
        by_kind[key] = by_kind.get(key, 0.0) + ms * 1e3
    weight_bytes = 2 * L.num_params(cfg) - 2 * cfg.vocab * cfg.d_model + 2 * cfg.d_model  # one embedding row
    kv_bytes = 2 * cfg.layers * 2 * cfg.heads * cfg.head_dim * (cfg.max_len + 1)  # cache read + new row
    step_bytes = weight_bytes + kv_bytes
    line = {
        "metric": "llama-like decode tokens/s (greedy, batch 1)",
        "value": round(steps / decode_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights 0.02*N(0,1) seed 0, random 512-token prompt seed 1)",
        "config": {"workload": C5_WORKLOAD,
                   "prefill_ms": round(prefill_s * 1e3, 3), "prefill_tokens_per_s": round(p / prefill_s, 1),
                   "setup_s": round(setup_s, 1), "weights_upload_ms": round(upload_s * 1e3, 1),
                   "weights_upload_gbps": round(upload_bytes / upload_s / 1e9, 1), "decode_step_hbm_bytes": step_bytes,
                   "decode_step_gbps": round(step_bytes / (ms_per_step / 1e3) / 1e9, 1),
                   "launch_units_per_step": sum(1 for n in names if n != "-"),
                   "gpu_us_per_step_by_kind": {kk: round(v, 2) for kk, v in sorted(by_kind.items())},
                   "gpu_us_per_step": round(sum(unit_ms) * 1e3, 2), "first_tokens": tokens[:8],
                   "graph": graph_stats, "all_graphs_ms_per_step": graph_ms,
                   "one_execute_ms_per_step": loop_ms, "one_execute_tokens_match": loop_match},
        "roofline": roofline(units, unit_ms, names, "bf16", C5_WORKLOAD),
    }
    line["roofline"]["traffic"] = traffic_from_profiles(C5_WORKLOAD, line["roofline"]["kernel"])
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_c5(cfg, weights, prompt, tokens)
    return line


C5_WORKLOAD = "llama_like_decode_8L_d2048_h16x128_ffn5632_v32000_prompt512"

# Keys of a secondary workload's line carried into the default run's line.
SUB_KEYS = ("metric", "value", "unit", "steps", "warmup", "ms_per_step", "higher_is_better", "dtype", "data",
            "config", "roofline", "cpu_baseline")


def bench_default(a) -> dict:
    """The driver's run (no --config): the headline C2 line (BASELINE.json
    configs[1], the fused-reduction half of the metric) with two more
    workloads measured in the same process and carried in the same JSON line:
    `c5`, the llama-like decode tokens/s (the metric's other half; always the
    config's 128 greedy tokens after the 512-token prompt, whatever --steps
    says), and `c1` (configs[0], the fused elementwise chain + row sum, timed
    over --steps executes). Each carries its own roofline (with the committed
    rocprof figure and HBM traffic) and CPU baseline."""
    import copy
    line = bench_program(a, WORKLOADS["c2"])
    sub1 = bench_program(copy.copy(a), WORKLOADS["c1"])
    line["c1"] = {k: sub1[k] for k in SUB_KEYS if k in sub1}
    a5 = copy.copy(a)
    a5.steps = 128
    a5.warmup = min(a.warmup, 10)
    sub5 = bench_c5(a5, extras=False)
    line["c5"] = {k: sub5[k] for k in SUB_KEYS if k in sub5}
    return line


def cpu_baseline_c5(cfg, weights, prompt, tokens, budget_s: float = 10.0) -> dict:
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
    return {"value": round(n / el, 3), "unit": "tokens/s", "cores": host_threads(), "kind": "port",
            "sample": f"{n} decode steps of the numpy oracle after the 512-token prefill "
                      f"({el / n * 1e3:.0f} ms/token, numpy matmul on all host threads)", "host": host_facts()}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 200; c3/c4 20; c5 128 tokens)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", choices=sorted(WORKLOADS) + ["c5"], default=None,
                    help="one workload; default: c2 as the line's value, with c5 and c1 carried in the same line")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {a.gpus}); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        return 2
    heavy = (a.config or "").startswith(("c3", "c4"))
    if a.steps is None:
        a.steps = 128 if a.config == "c5" else (20 if heavy else 200)
    if a.warmup is None:
        a.warmup = 10
    if a.config is None:
        line = bench_default(a)
    else:
        line = bench_c5(a) if a.config == "c5" else bench_program(a, WORKLOADS[a.config])
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
