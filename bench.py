"""Boundary-step throughput of minispeed_amd on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5]
                    [--workload gpt-1.3b | gpt-1.3b-shift3 | llama3-8b-shard | ...]
                    [--grad-dtype fp16] [--mode fused|materialize|contiguous] [--micro-batches 1]
                    [--zero-stage 1]
                    [--state-spacing-gib auto] [--no-cpu-baseline] [--copy-calibration]
                    [--hbm-ceilings]

A step is one gradient-accumulation boundary through the engine API
(``engine.step()``): the ragged-grad scan, the norm/clip/skip decision and
the fused AdamW + model cast, plus the one read-back of the step scalars and
the host bookkeeping.  Before each step one of two pre-generated gradient
sets, resident in HBM, is re-attached to ``param.grad`` (what the last
``backward`` of a window leaves).  The K timed steps run back to back,
bracketed as a whole by ``torch.cuda.synchronize()``; ``ms_per_step`` is
the bracket over K (so the first step's host work before its first kernel,
0.1-0.3 ms, adds that over K to each step: K defaults to 50).  The same steps are then run one at a time, each
bracketed on its own (``ms_per_step_synced``: the latency of one boundary,
host work before the first kernel included).  With ``--mode contiguous``
the accumulation kernels of the gradient hooks (backward work on the same
stream) run before every step, so its steps are only timed one at a time
(``timing`` in the JSON line says which).  A second, shorter run with
the masters and moments in separate allocations is reported next to the
engine's default placement (``separate_allocations``).

Workload (default): the 1.3B GPT-style buffer (24 layers, d 2048, vocab
50257, 292 ragged tensors, 1,315,723,264 params), fp16 gradients
N(0,1e-3) x 2^16 under the dynamic loss scale 2^16, fp32 masters N(0,0.02),
ZeRO-1 at world size 1, clip 1.0, AdamW (lr 1e-3, betas 0.9/0.999, eps 1e-8,
wd 0.01), WarmupDecayLR 100/1000.

Printed: one JSON line with Gparams/s as ``value``, whole-step HBM GB/s at
the algorithmic bytes per parameter, the dominant kernel's roofline (K3,
timed with HIP events on its own stream over the timed steps) and the CPU
baseline (the oracle's torch restatement of the reference step on this
host's cores, on a bounded sample of the same tensor list).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "boundary-step Gparams/s + HBM GB/s (% of peak) at 1.3B fp16, 1 GPU"
PEAK_GBPS = 8000.0
# HBM bytes per launch counted by two rocprofv3 --pmc runs of this file's
# default workload and layout (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0, both scales
# calibrated on a 1 GiB device copy in the same runs; mean of 10 launches);
# commands and per-kernel counts in profiles/traffic_gpt-1.3b_fp16.md.  Keyed
# by kernel / workload / grad dtype / mode / state window in GiB: a run in
# any other configuration reports null.
MEASURED_TRAFFIC = {
    "k3/gpt-1.3b/fp16/fused/36.0": 36_840_508_262,
    "k1/gpt-1.3b/fp16/fused/36.0": 2_639_900_128,
}

# algorithmic bytes per parameter: (K1, K3) for half / fp32 gradients
BYTES = {
    ("fused", 2): (2, 28),         # K1 read g2 | K3 read g2+p4+m4+v4, write p4+m4+v4+model2
    ("materialize", 2): (6, 30),   # K1 read g2 write f4 | K3 read f4+12, write 12+2
    ("fused", 4): (4, 32),
    ("materialize", 4): (8, 32),
    # contiguous: the accumulation kernel leaves the tile statistics, so the
    # boundary folds them (12 B per 2048 params) instead of a K1 read of the
    # fp32 sums | K3 read 4+12, write 12+2
    ("contiguous", 2): (0, 30),
    ("contiguous", 4): (0, 30),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _spacing(text: str):
    return "auto" if text == "auto" else float(text)


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="gpt-1.3b")
    ap.add_argument("--grad-dtype", default="fp16", choices=["fp16", "bf16", "fp32"])
    ap.add_argument("--mode", default="fused", choices=["fused", "materialize", "contiguous"])
    ap.add_argument("--micro-batches", type=int, default=1,
                    help="with --mode contiguous: gradient accumulation steps per window (the "
                         "hooks add each micro-batch's gradients into the fp32 sums)")
    ap.add_argument("--zero-stage", type=int, default=1, choices=[0, 1, 2, 3],
                    help="ZeRO stage at world size 1 (3: also times the parameter gather)")
    ap.add_argument("--stage3-gather-reuse", action="store_true",
                    help="hip_boundary.stage3_gather_reuse: the ZeRO-3 gather skips the cast "
                         "while the model buffer holds the cast of the current masters")
    ap.add_argument("--state-spacing-gib", type=_spacing, default="auto",
                    help="hip_boundary.state_spacing_gib of the engine: auto (the engine's default), "
                         "0 (separate allocations) or a window in GiB")
    ap.add_argument("--no-compare-separate", dest="compare_separate", action="store_false",
                    help="skip the second, shorter run with the state in separate allocations")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-timing", action="store_true",
                    help="time the steps without the per-kernel HIP events (no roofline)")
    ap.add_argument("--cpu-sample-params", type=int, default=0,
                    help="CPU baseline sample (0: the whole workload, ~1 minute at 1.3B)")
    ap.add_argument("--hbm-ceilings", action="store_true",
                    help="measure streaming-bandwidth reference points instead of the boundary step")
    ap.add_argument("--no-extra-workloads", dest="extra_workloads", action="store_false",
                    help="with the default headline workload: skip the short runs of the other "
                         "single-GPU configurations (GPT-2 124M, 350M, the Llama-3-8B shard)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device copy (a counter yardstick for rocprofv3 --pmc)")
    return ap.parse_args(argv)


def engine_config(grad_dtype: str, mode: str, zero_stage: int = 1, state_spacing_gib="auto",
                  gas: int = 1, gather_reuse: bool = False) -> dict:
    cfg = {
        "train_micro_batch_size_per_gpu": 1,
        "gradient_accumulation_steps": gas,
        "gradient_clipping": 1.0,
        "dtype": grad_dtype,
        "optimizer": {"type": "AdamW",
                      "params": {"lr": 1e-3, "betas": [0.9, 0.999], "eps": 1e-8, "weight_decay": 0.01}},
        "scheduler": {"type": "WarmupDecayLR",
                      "params": {"warmup_min_lr": 0.0, "warmup_max_lr": 1e-3,
                                 "warmup_num_steps": 100, "total_num_steps": 1000}},
        "zero_optimization": {"stage": zero_stage},
        "hip_boundary": {"materialize_flat_grad": mode == "materialize",
                         "contiguous_gradients": mode == "contiguous",
                         "state_spacing_gib": state_spacing_gib,
                         "stage3_gather_reuse": gather_reuse},
        "steps_per_print": 1000000,
    }
    if grad_dtype == "fp16":
        cfg["fp16"] = {"enabled": True, "loss_scale": 0, "initial_scale_power": 16,
                       "loss_scale_window": 1000}
    return cfg


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo", "r", encoding="utf-8") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(shapes, grad_dtype: str, sample_params: int) -> dict:
    """Time the oracle's torch restatement of the reference boundary step on
    the host cores: the whole tensor list (``sample_params <= 0``) or its
    leading transformer layers up to ``sample_params``."""
    import torch
    from torch import nn

    from oracle import boundary as ob

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    threads = max(1, min(threads, 16))
    torch.set_num_threads(threads)
    # the whole list, or whole transformer layers after the embeddings until
    # the sample size
    sample, total = [], 0
    for s in (shapes if sample_params <= 0 else shapes[2:]):
        if 0 < sample_params <= total:
            break
        n = 1
        for x in s:
            n *= x
        sample.append(s)
        total += n
    gen = torch.Generator().manual_seed(0)
    params = [nn.Parameter(torch.randn(*s, generator=gen) * 0.02) for s in sample]
    dt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[grad_dtype]
    eng = ob.Engine([params], [{"lr": 1e-3, "weight_decay": 0.01}], dtype=grad_dtype, zero_stage=1,
                    clip=1.0, initial_scale_power=16, scheduler="WarmupDecayLR",
                    scheduler_params={"warmup_max_lr": 1e-3, "warmup_num_steps": 100,
                                      "total_num_steps": 1000})
    mult = 2.0 ** 16 if grad_dtype == "fp16" else 1.0
    grads = [(torch.randn(*s, generator=gen) * 1e-3 * mult).to(dt) for s in sample]
    times = []
    for it in range(4):
        for p, g in zip(params, grads):
            p.grad = g
        eng.micro_steps += 1
        t0 = time.perf_counter()
        ok = eng.step()
        times.append(time.perf_counter() - t0)
        assert ok
    times = sorted(times[1:])
    med = times[len(times) // 2]
    what = ("the whole workload" if len(sample) == len(shapes)
            else "the leading transformer layers of the same list")
    return {
        "value": total / med / 1e9,
        "unit": "Gparams/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle torch-CPU restatement of the reference step on {len(sample)} tensors "
                   f"({total:,} params: {what}); median of 3 steps after 1 warm-up, "
                   f"{med * 1e3:.0f} ms/step; {threads} threads of {os.cpu_count()} on "
                   f"{cpu_model()}"),
        # effective GB/s at the fused path's 30 B/param and at the ~150
        # B/param the unfused torch sequence actually moves
        "gbps_at_30_bytes": round(30 * total / med / 1e9, 2),
        "gbps_at_150_bytes": round(150 * total / med / 1e9, 2),
    }


# the other single-GPU configurations: (workload, ZeRO stage) of the
# reported short runs next to the headline, with what they stand for
# (name, ZeRO stage, description, timed steps): about 50-100 ms of timed
# steps each, so that the start of the timed loop (the first step's host
# work before its first kernel) adds little to a step of 0.6 ms
EXTRA_WORKLOADS = (
    ("gpt2-124m", 2, "GPT-2 small (124M params, 148 tensors), fp16 grads x 2^16, ZeRO-2", 100),
    ("gpt-350m", 0, "350M GPT (24 layers, d 1024, 292 tensors), fp16 grads x 2^16, ZeRO-0", 50),
)
EXTRA_STEPS, EXTRA_WARMUP = 20, 5      # the Llama-3-8B shard (4.6 ms steps)


def extra_workloads(args, run_engine, gen, dev, gdt, mult) -> dict:
    """Short runs of the boundary step on the other single-GPU
    configurations, each through the engine with its default placement
    (step time back to back, kernel times from HIP events), and the
    Llama-3-8B shard at component level.  The bar of each is 80% of the
    8 TB/s peak at the bytes its step moves."""
    import numpy as np
    import torch

    from minispeed_amd.workloads import numel, shapes_of

    out = {}
    for name, stage, desc, steps in EXTRA_WORKLOADS:
        shapes = shapes_of(name)
        n = numel(shapes)
        sets = []
        old = args.zero_stage
        args.zero_stage = stage
        try:
            r = run_engine("auto", steps, True, shapes=shapes, grad_sets=sets, warmup=EXTRA_WARMUP)
        finally:
            args.zero_stage = old
        del sets
        torch.cuda.empty_cache()
        gbps = 30 * n / (r["ms_step"] * 1e-3) / 1e9
        out[name] = {"desc": desc, "params": n, "zero_stage": stage, "steps": steps,
                     "ms_per_step": round(r["ms_step"], 4),
                     "value": round(n / (r["ms_step"] * 1e-3) / 1e9, 3), "unit": "Gparams/s",
                     "hbm_gbps": round(gbps, 1), "hbm_frac": round(gbps / PEAK_GBPS, 4),
                     "bar_ms_at_80pct": round(30 * n / (0.8 * PEAK_GBPS * 1e9) * 1e3, 4),
                     "kernel_ms": {k: round(v, 4) for k, v in r["k_ms"].items()},
                     "k3_gbps": round(28 * n / (r["k_ms"]["k3"] * 1e-3) / 1e9, 1),
                     "state_placement": r["placement"]}
        log(f"[bench] {name}: {r['ms_step']:.4f} ms/step, {gbps:.0f} GB/s")
    shard_args = argparse.Namespace(**vars(args))
    shard_args.steps, shard_args.warmup = EXTRA_STEPS, EXTRA_WARMUP
    sh = bench_llama_shard(shard_args)
    s_params = sh["config"]["shard_params"]
    out["llama3-8b-shard"] = {
        "desc": sh["config"]["workload"], "params": s_params, "model_params": sh["config"]["model_params"],
        "steps": EXTRA_STEPS, "ms_per_step": sh["ms_per_step"], "value": sh["value"], "unit": "Gparams/s",
        "hbm_gbps": sh["hbm_gbps"], "hbm_frac": round(sh["hbm_gbps"] / PEAK_GBPS, 4),
        "bar_ms_at_80pct": round(30 * s_params / (0.8 * PEAK_GBPS * 1e9) * 1e3, 4),
        "kernel_ms": sh["kernel_ms"], "cast_on_gather": sh["cast_on_gather"]}
    torch.cuda.empty_cache()
    return out


def bench_llama_shard(args) -> dict:
    """One rank's 1/8 ZeRO-3 shard of Llama-3-8B (rank 3 of 8) plus the full
    cast-on-gather, at component level through the C ABI.

    The shard step runs K1 -> K2 -> K3 over the owned flat range with the
    reduce-scattered bf16 gradient pieces of every tensor that intersects it
    (ragged views of one buffer) and bf16 placeholders as cast targets; the
    gather casts a full fp32 master buffer into the 291 full-shaped bf16
    parameters (K4)."""
    import ctypes

    import numpy as np
    import torch

    from minispeed_amd import _native
    from minispeed_amd.boundary import HostReadback, LaunchTimer, adamw_params
    from minispeed_amd.flat import AUTO_SPACING, FlatLayout, check_table, state_buffers
    from minispeed_amd.workloads import shapes_of

    lib = _native.load()
    dev = torch.device("cuda", 0)
    stream = _native.stream_handle(dev)
    shapes = shapes_of("llama3-8b")
    numels = [int(np.prod(s)) for s in shapes]
    lay = FlatLayout(numels, rank=3, world_size=8, zero_stage=3)
    lo, hi = lay.shard_start, lay.shard_end
    S, N = hi - lo, lay.numel_padded
    log(f"[bench] llama3-8b: {len(shapes)} tensors, {N:,} params; rank 3 of 8 owns [{lo:,}, {hi:,})")
    gen = torch.Generator(device=dev).manual_seed(5)
    # the partitioned masters and the moments, placed as the engine places
    # them by default
    master, m, v = state_buffers([[S, S, S]], dev, AUTO_SPACING)[0]
    master.normal_(0.0, 0.02, generator=gen)
    # two gradient sets, taken in turn, as the 1.3B bench does (the same
    # buffer every step would let a step's scan find the previous scan's
    # last lines still in the Infinity Cache)
    grads = []
    for _ in range(2):
        grad = torch.empty(S, dtype=torch.bfloat16, device=dev)
        for a in range(0, S, 1 << 27):   # bounded fp32 temporaries
            b = min(S, a + (1 << 27))
            grad[a:b] = torch.randn(b - a, generator=gen, device=dev) * 1e-4
        grads.append(grad)
    holder = torch.empty(S, dtype=torch.bfloat16, device=dev)
    tables = []
    for grad in grads:
        gs, ms_ = [], []
        for off, n in zip(lay.offsets, numels):
            a, b = max(off, lo), min(off + n, hi)
            if b > a:
                gs.append((grad.data_ptr() + (a - lo) * 2, (a, b), 2))
                ms_.append((holder.data_ptr() + (a - lo) * 2, (a, b), 2))
            else:
                gs.append(None)
                ms_.append(None)
        table = lay.segments(lo, hi, gs, ms_)
        check_table(table, lo, hi)
        tables.append(torch.from_numpy(table).to(dev))
    nseg = int(tables[0].shape[0])
    nb = _native.stats_blocks()
    psum = torch.empty(nb, dtype=torch.float64, device=dev)
    pflag = torch.empty(nb, dtype=torch.int32, device=dev)
    ntiles = _native.scan_tiles(hi - lo)
    tsum = torch.empty(ntiles, dtype=torch.float64, device=dev)
    tflag = torch.empty(ntiles, dtype=torch.int32, device=dev)
    scal = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, device=dev)
    readback = HostReadback()
    timer = LaunchTimer()

    def step(k: int, timed: bool):
        """K1 -> K2 -> K3 with the engine's one host wait: for K2's scalars,
        written straight to pinned host memory, while K3 runs on."""
        t = timer if timed else None
        tdev = tables[k % 2]
        hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, k + 1)
        tok = t.start("k1") if t else None
        _native.check(lib.ms_grad_stats(tdev.data_ptr(), nseg, _native.DTYPE_BF16, lo, hi,
                                        lo, hi, 0, 1.0, None, tsum.data_ptr(), tflag.data_ptr(),
                                        ntiles, psum.data_ptr(), pflag.data_ptr(), nb, stream),
                      "ms_grad_stats")
        if t:
            t.stop(tok)
        readback.arm()
        _native.check(lib.ms_norm_clip(psum.data_ptr(), pflag.data_ptr(), nb, 1, 1, 1.0, 0, 1.0,
                                       0, 0, 1000, 1.0, 2.0 ** 24, scal.data_ptr(), readback.ptr,
                                       stream), "ms_norm_clip")
        tok = t.start("k3") if t else None
        _native.check(lib.ms_fused_adamw(master.data_ptr(), m.data_ptr(), v.data_ptr(), None,
                                         tdev.data_ptr(), nseg, _native.DTYPE_BF16,
                                         _native.DTYPE_BF16, lo, hi, ctypes.byref(hp),
                                         scal.data_ptr(), stream), "ms_fused_adamw")
        if t:
            t.stop(tok)
        return readback.wait(stream)

    for k in range(args.warmup):
        step(k, False)
    # the timed steps with nothing recorded between the kernels, then the
    # same steps again with HIP events around K1 and K3 for their times
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        last = [step(args.warmup + k, False)]
    torch.cuda.synchronize()
    step_s = [(time.perf_counter() - t0) / args.steps]
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(args.warmup + args.steps + k, True)
    torch.cuda.synchronize()
    ms_events = (time.perf_counter() - t0) / args.steps * 1e3
    res = last[0]
    # norm = sqrt(S * 1e-8) ~ 3.2 > clip 1.0: the clip path is exercised
    if res.overflow or not res.clip_applied:
        raise RuntimeError(f"unexpected step scalars: overflow={res.overflow} clip={res.clip_applied}")

    # cast-on-gather of the full model: fp32 masters (all ranks' shards) -> bf16 params
    del grads, grad, holder
    full = torch.randn(N, generator=gen, device=dev) * 0.02
    params16 = torch.empty(N, dtype=torch.bfloat16, device=dev)
    gtable = lay.segments(0, N, [None] * len(numels),
                          [(params16.data_ptr() + off * 2, (off, off + n), 2)
                           for off, n in zip(lay.offsets, numels)])
    check_table(gtable, 0, N)
    gdev = torch.from_numpy(gtable).to(dev)
    cast_ms = []
    for k in range(3 + args.steps):
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
        _native.check(lib.ms_cast_to_model(full.data_ptr(), 0, N, gdev.data_ptr(), len(gtable),
                                           _native.DTYPE_BF16, stream), "ms_cast_to_model")
        ev1.record()
        torch.cuda.synchronize()
        if k >= 3:
            cast_ms.append(ev0.elapsed_time(ev1))
    sample = torch.randint(0, N, (1 << 20,), device=dev)
    assert torch.equal(params16[sample], full[sample].to(torch.bfloat16))

    ms_step = float(np.mean(step_s)) * 1e3
    k3 = float(np.mean(timer.durations_ms("k3")))
    cast = float(np.mean(cast_ms))
    return {
        "metric": "Llama-3-8B 1/8 ZeRO-3 shard boundary step + full bf16 cast-on-gather, 1 GPU",
        "value": round(S / (ms_step * 1e-3) / 1e9, 3),
        "unit": "Gparams/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_with_kernel_events": round(ms_events, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: two sets of bf16 grads N(0,1e-4) taken in turn, fp32 masters N(0,0.02)",
        "config": {"workload": "one rank's 1/8 shard of Llama-3-8B (rank 3 of 8, fused mode)",
                   "shard_params": S, "model_params": N, "tensors": len(shapes),
                   "shard_segments": nseg, "bytes_per_param": 30},
        "hbm_gbps": round(30 * S / (ms_step * 1e-3) / 1e9, 1),
        "kernel_ms": {"k1": round(float(np.mean(timer.durations_ms("k1"))), 4), "k3": round(k3, 4),
                      "cast_on_gather": round(cast, 4)},
        "roofline": {"kernel": "K3 k_adamw (fused AdamW + placeholder cast)", "bound": "hbm",
                     "achieved": round(28 * S / (k3 * 1e-3) / 1e9, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(28 * S / (k3 * 1e-3) / 1e9 / PEAK_GBPS, 4),
                     "traffic": None, "bytes_per_param": 28},
        "cast_on_gather": {"ms": round(cast, 4), "params": N, "bytes_per_param": 6,
                           "gbps": round(6 * N / (cast * 1e-3) / 1e9, 1)},
        "cpu_baseline": None,
    }


def traffic_for(kernel: str, workload: str, grad_dtype: str, mode: str, spacing_gib: float):
    """HBM bytes per launch counted for this kernel, workload and state
    layout, or None where no counter runs were made for it."""
    return MEASURED_TRAFFIC.get(f"{kernel}/{workload}/{grad_dtype}/{mode}/{float(spacing_gib)}")


def bench_hbm_ceilings(args) -> dict:
    """What this GPU's HBM sustains for each mix of streams the boundary
    kernels use, measured with the streaming probes of libms_hbm_probe.so,
    independent of the boundary kernels: one read stream, one write stream,
    a copy, in-place read-modify-write of one and of three arrays (AdamW's
    p, m, v) and K3's whole mix (three read-modify-write arrays plus one read
    and one write array), 4 GiB per array, the arrays 32 GiB apart in one
    allocation (an arena of the kind the engine places its state in).  Each mix is run over a grid of launch
    shapes (threads per block, 16-byte vectors per lane, lane or wave order,
    non-temporal hints) and the fastest is reported; then K3 itself over
    2^30 elements in the same placement.  Median of 6 launches after 2, HIP
    events on the current stream; bytes are the algorithmic ones."""
    import ctypes

    import numpy as np
    import torch

    from minispeed_amd import _native
    from minispeed_amd.boundary import adamw_params

    dev = torch.device("cuda", 0)
    stream = _native.stream_handle(dev)
    probe = ctypes.CDLL(os.path.join(ROOT, "bench_probes", "libms_hbm_probe.so"))
    P = ctypes.c_void_p
    probe.msp_stream.restype = ctypes.c_int
    probe.msp_stream.argtypes = [ctypes.POINTER(P), ctypes.c_int32, ctypes.POINTER(P), ctypes.c_int32,
                                 ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                 ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, P, P]
    gib = 1 << 30
    nbytes = 4 * gib
    arena = torch.empty(4 * 32 * gib + nbytes, dtype=torch.uint8, device=dev)
    base = arena.data_ptr()
    at = [base + k * 32 * gib for k in range(5)]
    for a in at:
        assert a + nbytes <= base + arena.numel()
    for k in range(5):
        arena[k * 32 * gib:k * 32 * gib + nbytes].fill_(1)
    sink = torch.zeros(1024, dtype=torch.int32, device=dev)

    def median_ms(fn, reps=6, warm=2):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        evs = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            evs.append((a, b))
        torch.cuda.synchronize()
        return float(np.median([a.elapsed_time(b) for a, b in evs]))

    mixes = {
        "read": ([at[0]], []), "write": ([], [at[0]]), "copy": ([at[0]], [at[1]]),
        "rmw_1_array": ([at[0]], [at[0]]),
        "rmw_3_arrays": (at[:3], at[:3]),
        "k3_mix": (at[:4], at[:3] + [at[4]]),
        # K1 writing the fp32 flat gradient and K5's first micro-batch
        # (read 2, write 4 B/element), K4 (read 4, write 2) and K5's later
        # micro-batches (read 2 + 4, write 4)
        "read_1_write_2": ([at[0]], at[1:3]),
        "read_2_write_1": (at[:2], [at[2]]),
        "read_3_write_2": (at[:3], at[3:5]),
    }
    out = {}
    for name, (rd, wr) in mixes.items():
        rdp = (P * 4)(*rd, *([0] * (4 - len(rd))))
        wrp = (P * 4)(*wr, *([0] * (4 - len(wr))))
        best = None
        for threads in (128, 256):
            for unroll in (1, 2, 4):
                for wave in (0, 1):
                    for ntl, nts in ((1, 1), (1, 0), (0, 1), (0, 0)):
                        if (not rd and ntl) or (not wr and nts):
                            continue

                        def fn():
                            rc = probe.msp_stream(rdp, len(rd), wrp, len(wr), nbytes // 16, threads, unroll,
                                                  wave, 0, ntl, nts, sink.data_ptr(), stream)
                            if rc != 0:
                                raise RuntimeError(f"msp_stream failed with {rc}")
                        ms = median_ms(fn)
                        if best is None or ms < best["ms"]:
                            best = {"ms": round(ms, 4), "threads": threads, "unroll": unroll,
                                    "order": "wave" if wave else "lane", "nt_load": ntl, "nt_store": nts}
        best["gbps"] = round(nbytes * (len(rd) + len(wr)) / (best["ms"] * 1e-3) / 1e9, 1)
        out[name] = best
        log(f"[bench] {name}: {best['gbps']:.0f} GB/s ({best})")

    # K3's access pattern (AdamW arithmetic, fp16 g and copy) on layouts of
    # the state: p, m, v in three 32 GiB windows of one allocation, the
    # same with XCD-ordered blocks, and the three interleaved per tile of T
    # elements in one array
    probe.msp_adam_layout.restype = ctypes.c_int
    probe.msp_adam_layout.argtypes = [ctypes.POINTER(P), P, P, ctypes.c_int64, ctypes.c_int32,
                                      ctypes.c_int32, P]
    n_el = nbytes // 4
    arena[:3 * nbytes].zero_()           # room for the interleaved state in window 0
    layouts = {"windows": ([at[0], at[1], at[2]], 0, 0),
               "windows_xcd_1024": ([at[0], at[1], at[2]], 0, 1024),
               "interleaved_512": ([at[0]] * 3, 512, 0),
               "interleaved_2048": ([at[0]] * 3, 2048, 0)}
    k3_layout = {}
    for name, (state, inter, chunk) in layouts.items():
        sp = (P * 3)(*state)

        def fn():
            rc = probe.msp_adam_layout(sp, at[3], at[4], n_el, inter, chunk, stream)
            if rc != 0:
                raise RuntimeError(f"msp_adam_layout failed with {rc}")
        ms = median_ms(fn)
        k3_layout[name] = {"ms": round(ms, 4), "gbps": round(28 * n_el / (ms * 1e-3) / 1e9, 1)}
        log(f"[bench] K3 layout {name}: {ms:.4f} ms")
    out["k3_layout"] = dict(k3_layout, note=f"{n_el} elements, 28 B each")

    lib = _native.load()
    n = 1 << 30
    g = torch.full((n,), 0.5, dtype=torch.float16, device=dev)
    model = torch.empty(n, dtype=torch.float16, device=dev)
    tab = torch.tensor([[0, n, g.data_ptr(), model.data_ptr()]], dtype=torch.int64, device=dev)
    hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, 10)
    clean = torch.zeros(_native.SCALARS_BYTES, dtype=torch.uint8, device=dev)

    def k3():
        _native.check(lib.ms_fused_adamw(at[0], at[1], at[2], None, tab.data_ptr(), 1, _native.DTYPE_F16,
                                         _native.DTYPE_F16, 0, n, ctypes.byref(hp), clean.data_ptr(),
                                         stream), "ms_fused_adamw")
    ms = median_ms(k3)
    out["k3_adamw"] = {"ms": round(ms, 4), "gbps": round(28 * n / (ms * 1e-3) / 1e9, 1),
                       "note": "2^30 elements, fp16 grads and model copy in separate allocations"}
    log(f"[bench] K3: {out['k3_adamw']['gbps']:.0f} GB/s")
    return {"hbm_ceilings": out, "bytes_per_array": nbytes, "peak_gbps": PEAK_GBPS,
            "placement": "arrays 32 GiB apart in one allocation"}


def main(argv=None) -> int:
    args = parse(argv)
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: bench.py measures the boundary step on one "
                                   "GPU; multi-GPU runs are not part of it"}))
        return 2
    if args.micro_batches < 1 or (args.micro_batches > 1 and args.mode != "contiguous"):
        print(json.dumps({"error": "--micro-batches > 1 applies to --mode contiguous only: in the "
                                   "other modes micro-batches accumulate in autograd, outside "
                                   "the boundary step"}))
        return 2
    import numpy as np
    import torch
    from torch import nn

    import minispeed_amd as ms
    from minispeed_amd.boundary import LaunchTimer
    from minispeed_amd.workloads import WORKLOADS, numel, shapes_of

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        return 1
    if args.hbm_ceilings:
        torch.cuda.set_device(0)
        print(json.dumps(bench_hbm_ceilings(args)), flush=True)
        return 0
    if args.workload == "llama3-8b-shard":
        torch.cuda.set_device(0)
        print(json.dumps(bench_llama_shard(args)), flush=True)
        return 0
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    shapes = shapes_of(args.workload)
    n_params = numel(shapes)
    gdt = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[args.grad_dtype]
    log(f"[bench] workload {args.workload}: {len(shapes)} tensors, {n_params:,} params, "
        f"grads {args.grad_dtype}, mode {args.mode}")
    gen = torch.Generator(device=dev).manual_seed(1234)
    mult = 2.0 ** 16 if args.grad_dtype == "fp16" else 1.0
    grad_sets = []

    def run_engine(spacing, steps: int, kernel_timing: bool, shapes=shapes, grad_sets=grad_sets,
                   warmup: int = args.warmup) -> dict:
        """Build an engine with this state placement, warm it up and time
        ``steps`` boundaries back to back and then one at a time.  As in
        training, the engine (and its state) is built before the gradients
        exist; two gradient sets are made once and shared by every run of
        one tensor list."""
        params = [nn.Parameter(torch.randn(*s, generator=gen, device=dev) * 0.02) for s in shapes]
        module = nn.ParameterList(params)
        engine = ms.initialize(model=module, model_parameters=list(module),
                               config=engine_config(args.grad_dtype, args.mode, args.zero_stage, spacing,
                                                    args.micro_batches,
                                                    gather_reuse=args.stage3_gather_reuse))
        while len(grad_sets) < 2:
            grad_sets.append([(torch.randn(*s, generator=gen, device=dev) * (1e-3 * mult)).to(gdt)
                              for s in shapes])
        where = engine.state_placement
        window = where.window / 2 ** 30
        torch.cuda.synchronize()
        log(f"[bench] state placement {spacing!r}: window {window:g} GiB, {where}; warming up")
        gather_s, accum_s = [], []   # accum_s: (micro-batch index, seconds)

        def attach(k: int, measure: bool = False) -> None:
            """What the last backward of a window leaves: grads on every param
            (ZeRO-3: after the forward's parameter gather; contiguous mode:
            after the post-accumulate-grad hooks and their end-of-backward
            flush).  With ``measure`` the gather and the hooks are timed on
            their own, between synchronisations."""
            if args.zero_stage == 3:
                if measure:
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                engine.optimizer.gather_parameters()
                if measure:
                    torch.cuda.synchronize()
                    gather_s.append(time.perf_counter() - t0)
            if engine.contiguous is None:
                for p, g in zip(params, grad_sets[k % 2]):
                    p.grad = g
                engine.micro_steps += 1
                return
            for m in range(args.micro_batches):
                for p, g in zip(params, grad_sets[(k + m) % 2]):
                    p.grad = g
                if measure:
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                for i, p in enumerate(params):
                    engine.contiguous.accumulate(0, i, p)
                engine.contiguous.flush()
                if measure:
                    torch.cuda.synchronize()
                    accum_s.append((m, time.perf_counter() - t0))
                engine.micro_steps += 1

        def boundary() -> None:
            if not engine.step():
                raise RuntimeError("boundary step was skipped (unexpected overflow)")

        for k in range(warmup):
            attach(k)
            boundary()
        torch.cuda.synchronize()
        gather_s.clear()
        accum_s.clear()
        # 2 events per kernel launch (K1 and K3 per group, K2 once), created
        # before the timed loop
        timer = LaunchTimer(reserve=2 * (2 * len(engine.flat_groups) + 1) * steps)
        # Contiguous mode: the hooks' accumulation kernels are backward work
        # on the same stream, so its boundaries are timed one at a time (the
        # second loop) and the kernel events go there.
        back_to_back = engine.contiguous is None
        elapsed = elapsed_events = None
        if back_to_back:
            # the timed steps, bracketed as a whole: each step re-attaches its
            # gradients (what the window's last backward leaves) and runs the
            # boundary; the host work of step k+1 overlaps K3 of step k.
            # Nothing is recorded between the kernels here.
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for k in range(steps):
                attach(k)
                boundary()                       # ends with the one scalar read-back
            torch.cuda.synchronize()
            elapsed = time.perf_counter() - t0
            if kernel_timing:
                # the same steps again with a HIP event before and after every
                # launch, for the kernel durations; each event puts a few
                # microseconds between two kernels, so this pass is slower by
                # up to ~30 us per step and gives the kernel times only
                engine.optimizer.launch_timer = timer
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for k in range(steps):
                    attach(k)
                    boundary()
                torch.cuda.synchronize()
                elapsed_events = time.perf_counter() - t0
                engine.optimizer.launch_timer = None
        # the same steps one at a time, each bracketed by synchronisations: the
        # latency of one boundary, host work before K1 included
        step_s = []
        for k in range(steps):
            attach(k, measure=True)
            if not back_to_back:
                engine.optimizer.launch_timer = timer if kernel_timing else None
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            boundary()
            torch.cuda.synchronize()
            step_s.append(time.perf_counter() - t1)
            engine.optimizer.launch_timer = None
        if elapsed is None:
            elapsed = sum(step_s)
        log(f"[bench] {steps} boundary steps: {elapsed * 1e3:.3f} ms "
            f"{'back to back' if back_to_back else 'one at a time'}, "
            f"{sum(step_s) * 1e3:.3f} ms one at a time")
        out = {"ms_step": elapsed / steps * 1e3, "step_s": step_s, "window_gib": window,
               "ms_step_events": (elapsed_events / steps * 1e3 if elapsed_events is not None
                                  else None),
               "placement": {"arena_gib": round(where.arena_bytes / 2 ** 30, 3),
                             "held_gib": round(where.held_bytes / 2 ** 30, 3),
                             "returned_to_allocator_gib": round(where.returned_bytes / 2 ** 30, 3)},
               "timing": "back to back" if back_to_back else "one at a time",
               "k_ms": ({k: float(np.mean(timer.durations_ms(k))) for k in ("k1", "k2", "k3")}
                        if kernel_timing else None)}
        if accum_s:
            first = [t for m, t in accum_s if m == 0]
            later = [t for m, t in accum_s if m > 0]
            out["accumulate_ms"] = {"first": float(np.mean(first)) * 1e3,
                                    "later": float(np.mean(later)) * 1e3 if later else None}
        if args.zero_stage == 3:
            # the gather is a change of views; a stale copy would cost one cast
            engine.optimizer.gather_parameters()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for g in engine.flat_groups:
                g.copy_flat_to_model()
            torch.cuda.synchronize()
            out["zero3"] = {"gather_ms": round(float(np.mean(gather_s)) * 1e3, 4),
                            "recast_ms": round((time.perf_counter() - t0) * 1e3, 4)}
        for p in params:
            p.grad = None
        del engine, module, params
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        return out

    head = run_engine(args.state_spacing_gib, args.steps, not args.no_kernel_timing)
    if args.copy_calibration:
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev)   # 1 GiB
        dst = torch.empty_like(src)
        src.fill_(1.0)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log("[bench] copy calibration: 3 x 1 GiB device copies (read 1 GiB + write 1 GiB each)")
    # the same workload with the masters and moments in three separate
    # allocations, for comparison with the placement above
    other = None
    if args.compare_separate and head["window_gib"] > 0:
        other = run_engine(0, max(5, args.steps // 2), not args.no_kernel_timing)

    ms_step = head["ms_step"]
    esize = 4 if args.grad_dtype == "fp32" else 2
    b1, b3 = BYTES[(args.mode, esize)]
    k_ms = head["k_ms"]
    step_gbps = (b1 + b3) * n_params / (ms_step * 1e-3) / 1e9
    traffic = traffic_for("k3", args.workload, args.grad_dtype, args.mode, head["window_gib"])
    result = {
        "metric": METRIC,
        "value": round(n_params / (ms_step * 1e-3) / 1e9, 3),
        "unit": "Gparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "timing": head["timing"],
        # the kernel-timing pass (same steps, HIP events around every launch)
        "ms_per_step_with_kernel_events": (round(head["ms_step_events"], 4)
                                           if head["ms_step_events"] is not None else None),
        "ms_per_step_synced": round(float(np.mean(head["step_s"])) * 1e3, 4),
        "ms_per_step_synced_median": round(float(np.median(head["step_s"])) * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": (f"synthetic: seeded {args.grad_dtype} grads N(0,1e-3)"
                 + (" x 2^16" if args.grad_dtype == "fp16" else "") + ", fp32 masters N(0,0.02)"),
        "config": {
            "workload": WORKLOADS[args.workload]["desc"],
            "params": n_params,
            "tensors": len(shapes),
            "grad_dtype": args.grad_dtype,
            "model_dtype": args.grad_dtype,
            "zero_stage": args.zero_stage,
            "stage3_gather_reuse": bool(args.stage3_gather_reuse and args.zero_stage == 3),
            "world_size": 1,
            "mode": args.mode,
            "state_spacing_gib": args.state_spacing_gib,
            "state_window_gib": head["window_gib"],
            "state_placement": head["placement"],
            "clip": 1.0,
            "bytes_per_param": b1 + b3,
        },
        "hbm_gbps": round(step_gbps, 1),
        "hbm_frac": round(step_gbps / PEAK_GBPS, 4),
        "kernel_ms": {k: round(v, 4) for k, v in k_ms.items()} if k_ms else None,
        "roofline": None,
        "cpu_baseline": None,
    }
    if k_ms:
        k3_gbps = b3 * n_params / (k_ms["k3"] * 1e-3) / 1e9
        result["roofline"] = {
            "kernel": "K3 k_adamw (fused AdamW + model cast)",
            "bound": "hbm",
            "achieved": round(k3_gbps, 1),
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(k3_gbps / PEAK_GBPS, 4),
            "traffic": traffic,
            "bytes_per_param": b3,
        }
    if other is not None:
        result["separate_allocations"] = {
            "ms_per_step": round(other["ms_step"], 4),
            "value": round(n_params / (other["ms_step"] * 1e-3) / 1e9, 3),
            "hbm_frac": round((b1 + b3) * n_params / (other["ms_step"] * 1e-3) / 1e9 / PEAK_GBPS, 4),
            "kernel_ms": ({k: round(v, 4) for k, v in other["k_ms"].items()} if other["k_ms"] else None),
        }
    if "accumulate_ms" in head:
        acc = head["accumulate_ms"]
        result["contiguous"] = {
            "micro_batches": args.micro_batches,
            # the hooks of one micro-batch: the first of a window writes the
            # fp32 sums (6 B/param), the later ones add into them (10 B/param)
            "accumulate_ms_first_micro_batch": round(acc["first"], 4),
            "accumulate_ms_later_micro_batch": (round(acc["later"], 4)
                                                if acc["later"] is not None else None)}
    if "zero3" in head:
        result["zero3"] = head["zero3"]
    if args.extra_workloads and args.workload == "gpt-1.3b" and args.mode == "fused" \
            and args.zero_stage == 1 and args.grad_dtype == "fp16" and args.state_spacing_gib == "auto":
        # the other single-GPU configurations, short runs of the same step
        del grad_sets[:]
        torch.cuda.empty_cache()
        result["workloads"] = extra_workloads(args, run_engine, gen, dev, gdt, mult)
    if not args.no_cpu_baseline:
        del grad_sets
        torch.cuda.empty_cache()
        log("[bench] CPU baseline (oracle restatement on host cores)")
        result["cpu_baseline"] = cpu_baseline(shapes, args.grad_dtype, args.cpu_sample_params)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
