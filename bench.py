#!/usr/bin/env python3
"""Batch-1 decode benchmark of the fused HIP decode step (one MI355X).

A step is one decode token of the configured model (default: the
Llama-3.2-1B-shaped fp32 model, BASELINE cfg 2: 64-token prompt, then greedy
decode).  Weights are seeded N(0, 0.02) synthetic weights in the reference's
.bin layout, generated on the host and uploaded once; the prompt and
`--warmup` decode steps run untimed, then exactly `--steps` decode steps are
timed with HIP events on the engine's stream, with a stream synchronisation
on both sides.  Prints one JSON line.

  value          decode tok/s (whole job: one GPU)
  achieved_GBps  algorithmic HBM bytes of the timed steps / time
  roofline       the dominant kernel: in the default persistent mode the
                 whole-token kernel k_decode_persistent (one launch = one
                 decode step, so its bytes are the step's algorithmic bytes
                 and its average launch duration over the timed region is the
                 region's HIP-event time per step; the per-launch events of
                 --profile-steps more steps are reported beside it); in --mode
                 multi the W1/W3 + SwiGLU GEMV, timed with HIP events around
                 each of its launches in the profile steps
  prefill        the batched prompt prefill of cfg 5 (Qwen3-4B shape, 512
                 tokens) on the matrix cores: prompt tok/s, algorithmic
                 TFLOP/s, the fraction of its matrix-core roofline (fp32
                 projections as six bf16 products each at the bf16 peak,
                 attention at the fp32 peak), and the MFMA-busy fraction
                 rocprofv3 measured for the same command
                 (profiles/prefill_qwen3_4b_pmc.txt)
  configs        the other four BASELINE configs, each a short decode leg of
                 its own workload (prompt via the batched prefill, then
                 --config-steps timed steps): tok/s, ms per step, GB/s and the
                 fraction of 8 TB/s, plus the prompt's prefill time
  hbm_measured   this box's HBM read and copy rates (kl_hbm_probe, outside the
                 timed region) and the decode rate as a fraction of the read rate
  cpu_baseline   the CPU oracle (a restatement of the reference CPU path,
                 "port") on the same workload: the same prompt through the
                 demo/main.cpp loop, then the timed positions (continued until
                 a bounded sample of CPU time is reached), on all the
                 process's host threads, plus a 1-thread figure
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
METRIC = "batch-1 decode tok/s + achieved HBM GB/s (% of peak), Llama-3.2-1B fp32"


def dominant_kernel_bytes(cfg) -> int:
    """Algorithmic bytes of one W1/W3+SwiGLU launch: both weight matrices
    (plus their int8 scales), the RMSNorm weight and residual read, h written."""
    D, F = cfg.dim, cfg.hidden_dim
    if cfg.quant:
        w = 2 * (F * D + (F * D // cfg.group_size) * 4)
    else:
        w = 2 * F * D * 4
    return w + 2 * D * 4 + F * 4


def measured_traffic(kernel: str, config: str, mode: str):
    """HBM bytes per launch of `kernel` on `config` in `mode`, as recorded by
    the rocprofv3 PMC summaries under profiles/ (FETCH_SIZE + WRITE_SIZE,
    calibrated against a copy kernel of known size).  The counters cannot be
    read in the same run as the timing, so the figure comes from those
    committed runs of this same command; None when no summary covers it."""
    pat = re.compile(r"measured: kernel=(\S+) config=(\S+) mode=(\S+) "
                     r"traffic_bytes_per_launch=(\d+)")
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None, None
    for name in sorted(os.listdir(pdir)):
        if not name.endswith("_pmc.txt"):
            continue
        with open(os.path.join(pdir, name)) as f:
            for line in f:
                m = pat.search(line)
                if m and m.group(1) == kernel and m.group(2) == config and m.group(3) == mode:
                    return int(m.group(4)), "profiles/" + name
    return None, None


MFMA_FP32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0


def measured_mfma_busy(config: str):
    """MFMA-busy fraction of the prefill kernels on `config`, from the
    committed rocprofv3 PMC summary of this same command
    (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs, per kernel,
    weighted by kernel time); None when no summary covers it."""
    pat = re.compile(r"measured: prefill config=(\S+) mfma_busy=([0-9.]+) gemm_mfma_busy=([0-9.]+) "
                     r"attn_mfma_busy=([0-9.]+)")
    path = os.path.join(ROOT, "profiles", f"prefill_{config}_pmc.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            m = pat.search(line)
            if m and m.group(1) == config:
                return {"all": float(m.group(2)), "gemm": float(m.group(3)),
                        "attention": float(m.group(4)),
                        "source": os.path.relpath(path, ROOT)}
    return None


def measure_prefill(K, cfg, eng=None, reps: int = 3) -> dict:
    """Batched prefill of the config's prompt (kl_engine_prefill), device time
    from HIP events inside the call; best of `reps` after one warm-up.
    `tflops` counts the algorithmic fp32 flops.  The roofline is the time the
    matrix cores would need at their peaks: fp32 projections run as six bf16
    products per multiply-add (kl_gemm_x6) at the bf16 peak; int8 ones on
    prompts of at most 32 rows (kl_gemm_q8s) as three bf16 products, or the
    int8 weight bytes at 8 TB/s where that is longer; other int8 ones, the
    attention and the classifier at the fp32 peak; `frac` = that time over
    the measured one."""
    if eng is None:
        eng = K.Engine(K.synth_image(cfg), cfg)
    prompt = K.prompt_tokens(cfg)
    P = len(prompt)
    eng.prefill(prompt, want_logits=False)
    times = [eng.prefill(prompt, want_logits=False)[2] for _ in range(reps)]
    ms = min(times)
    proj, attn, cls = cfg.prefill_flops_parts(P)
    fl = proj + attn + cls
    tf = fl / (ms / 1e3) / 1e12
    fp32_gemm = os.environ.get("KL_PREFILL_GEMM") == "f32"
    x6 = not cfg.quant and not fp32_gemm
    q8s = cfg.quant and not fp32_gemm and P <= 32 and cfg.group_size in (32, 64)
    if x6:
        gemm, proj_ms = "bf16x6 split products, fp32 accumulate", 6 * proj / MFMA_BF16_PEAK_TFLOPS / 1e9
    elif q8s:
        # three bf16 products per multiply-add, or the int8 weight bytes at 8 TB/s
        D, Dq, Dkv, F, L = cfg.dim, cfg.qd, cfg.kv_dim, cfg.hidden_dim, cfg.layers
        mats = L * (Dq * D + 2 * Dkv * D + D * Dq + 3 * F * D)
        wbytes = mats + mats // cfg.group_size * 4
        gemm = "int8 weights x bf16x3 activations (k_gemm_q8s), fp32 accumulate"
        proj_ms = max(3 * proj / MFMA_BF16_PEAK_TFLOPS / 1e9, wbytes / HBM_PEAK_GBPS / 1e6)
    else:
        gemm, proj_ms = "fp32 MFMA" + (" (int8 dequantised)" if cfg.quant else ""), proj / MFMA_FP32_PEAK_TFLOPS / 1e9
    roof_ms = proj_ms + (attn + cls) / MFMA_FP32_PEAK_TFLOPS / 1e9
    return {"config": cfg.name, "tokens": P, "ms": round(ms, 3),
            "tok_s": round(P / (ms / 1e3), 1), "tflops": round(tf, 2), "flops": int(fl),
            "gemm": gemm,
            "bound": "mfma", "roofline_ms": round(roof_ms, 3), "frac": round(roof_ms / ms, 4),
            "peak_tflops": {"bf16": MFMA_BF16_PEAK_TFLOPS, "fp32": MFMA_FP32_PEAK_TFLOPS},
            "dtype": "int8w-f32" if cfg.quant else "f32", "mfma_busy": measured_mfma_busy(cfg.name)}


# The other BASELINE configs, each timed as a short decode leg of its own
# workload (bench lines are cfg 2's; these ride along in "configs").
OTHER_CONFIGS = ("llama2_110m", "llama2_7b_q8", "qwen25_15b", "qwen3_4b")


def decode_leg(K, cfg, steps: int, warmup: int, prefill_reps: int) -> dict:
    """One config's workload: its prompt through the batched prefill (cfg 4:
    the 4000-position cache fill), `warmup` untimed decode steps (the first
    sampled by the prefill), then `steps` decode steps timed with HIP events
    on the engine's stream; then the prefill alone, best of `prefill_reps`."""
    t0 = time.time()
    img = K.synth_image(cfg)
    eng = K.Engine(img, cfg)
    t_setup = time.time() - t0
    eng.set_prefill(True)
    prompt = K.prompt_tokens(cfg)
    P = len(prompt)
    warmup = max(1, min(warmup, cfg.seq_len - P - steps + 1))
    toks, ms = eng.bench(prompt, warmup, steps)
    first_pos = P - 1 + warmup
    b = cfg.decode_bytes(first_pos, steps)
    gbps = b / (ms / 1e3) / 1e9
    out = {"config": cfg.name,
           "workload": f"{P}-token prompt (batched prefill), then {steps} timed greedy decode steps "
                       f"at positions {first_pos}..{first_pos + steps - 1}",
           "dtype": "int8w-f32" if cfg.quant else "f32",
           "tok_s": round(steps / (ms / 1e3), 2), "ms_per_step": round(ms / steps, 5),
           "achieved_GBps": round(gbps, 1), "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
           "bytes_per_token": int(b / steps), "mode": "persistent" if eng.mode == K.MODE_PERSISTENT
           else "multi"}
    if prefill_reps > 0:
        out["prefill"] = measure_prefill(K, cfg, eng, prefill_reps)
    print(f"# leg {cfg.name}: setup {t_setup:.1f} s; {out}", file=sys.stderr, flush=True)
    del eng, img
    return out


def host_cpu() -> dict:
    """Host threads visible to this process and the CPU model name."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": nproc, "model": model}


def cpu_baseline(K, cfg, img, first_pos: int, steps: int, gpu_tokens, seconds: float,
                 seconds_1t: float) -> dict:
    """The oracle (the reference CPU path restated) on the bench workload:
    the same prompt through the demo/main.cpp loop (prompt positions, then
    greedy decode) untimed up to the GPU's first timed position, then the
    GPU's timed positions, continued greedily until `seconds` of CPU time (at
    least `steps` steps) on every host thread the process may use; then a few
    more steps on 1 thread.  Also reports whether its greedy tokens over the
    GPU's positions equal the GPU's."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    hc = host_cpu()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or hc["nproc"]
    O.set_threads(threads)
    m = O.Model(img, cfg.family, cfg.quant)
    prompt = [int(t) for t in K.prompt_tokens(cfg)]
    P = len(prompt)
    seq = list(prompt)
    pos = 0
    t_fill = time.perf_counter()
    while pos < first_pos:  # positions 0 .. first_pos - 1, untimed
        lg = m.step(seq[pos], pos)
        if pos >= P - 1:
            seq.append(O.argmax(lg))
        pos += 1
    t_fill = time.perf_counter() - t_fill
    reserve = 8  # positions kept for the 1-thread leg
    n, t0 = 0, time.perf_counter()
    el = 0.0
    while pos < cfg.seq_len - 1 - reserve or n < steps:
        lg = m.step(seq[pos], pos)
        seq.append(O.argmax(lg))
        pos += 1
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= steps:
            break
    all_core = n / el
    last_all = pos - 1
    O.set_threads(1)
    n1, t1 = 0, time.perf_counter()
    el1 = 0.0
    while pos < cfg.seq_len - 1:
        lg = m.step(seq[pos], pos)
        seq.append(O.argmax(lg))
        pos += 1
        n1 += 1
        el1 = time.perf_counter() - t1
        if el1 >= seconds_1t and n1 >= 2:
            break
    O.set_threads(threads)
    # seq[i + 1] is the token sampled at position i (i >= P - 1); the GPU's
    # gpu_tokens[j] was sampled at position P - 1 + j.
    cpu_tok = seq[P:P + len(gpu_tokens)]
    return {
        "value": round(all_core, 4),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "value_1thread": round(n1 / el1, 4) if n1 else None,
        "host": hc,
        "tokens_match_gpu": [int(t) for t in gpu_tokens] == cpu_tok,
        "sample": f"{P}-token prompt and decode to position {first_pos - 1} untimed "
                  f"({t_fill:.1f} s), then {n} greedy decode steps at positions "
                  f"{first_pos}..{last_all} in {el:.1f} s on {threads} OpenMP threads "
                  f"({hc['nproc']} visible, {hc['model']}), then {n1} steps at positions "
                  f"{last_all + 1}..{pos - 1} in {el1:.1f} s on 1 thread",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0, help="timed decode steps (default: config)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="llama32_1b")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU baseline: timed seconds on all host threads")
    ap.add_argument("--cpu-seconds-1t", type=float, default=6.0,
                    help="CPU baseline: timed seconds on 1 thread")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-hbm-probe", action="store_true",
                    help="skip the on-box HBM read/copy bandwidth probe (kl_hbm_probe)")
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--mode", choices=("persistent", "multi"), default="persistent")
    ap.add_argument("--prefill-config", default="qwen3_4b",
                    help="also time the batched prefill of this config's prompt (default "
                         "qwen3_4b: 512 tokens) and report it under 'prefill'; 'none' skips it")
    ap.add_argument("--configs", default=",".join(OTHER_CONFIGS),
                    help="comma-separated configs timed as short decode legs of their own "
                         "workloads under 'configs' (prompt via the batched prefill); 'none' skips")
    ap.add_argument("--config-steps", type=int, default=32, help="timed decode steps per config leg")
    ap.add_argument("--config-warmup", type=int, default=8, help="untimed decode steps per config leg")
    ap.add_argument("--skip-decode", action="store_true",
                    help="run only the prefill leg (for profiling it); prints no bench line")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="first run one 256 MiB device-to-device copy, the known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is designed but not built)", file=sys.stderr)
        return 2

    import kuiperllama_amd as K

    if K.device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    if args.pmc_calibration:
        n = 64 << 20
        src, dst = K.DeviceArray(n, zero=True), K.DeviceArray(n)
        K.check(K.lib.kl_memcpy_d2d(dst.ptr, src.ptr, src.nbytes, None), "kl_memcpy_d2d")
        K.check(K.lib.kl_device_sync(), "kl_device_sync")
        src.free()
        dst.free()
    if args.skip_decode:
        if args.prefill_config == "none":
            print("bench.py: --skip-decode needs a prefill config", file=sys.stderr)
            return 2
        pf = measure_prefill(K, K.BASELINE[args.prefill_config])
        print(f"# prefill {pf}", file=sys.stderr, flush=True)
        return 0
    cfg = K.BASELINE[args.config]
    steps = args.steps or cfg.decode_steps
    P = cfg.prompt_len
    if P + args.warmup + steps - 1 > cfg.seq_len:
        # cfg 4 (4000-token prompt, 96 steps, seq_len 4096): fewer warmup steps
        warm = max(0, cfg.seq_len - P - steps + 1)
        if P + warm + steps - 1 > cfg.seq_len:
            print("bench.py: prompt + steps exceed the model's seq_len", file=sys.stderr)
            return 1
        print(f"# warmup {args.warmup} -> {warm} steps (seq_len {cfg.seq_len})", file=sys.stderr)
        args.warmup = warm
    t0 = time.time()
    img = K.synth_image(cfg)
    t_img = time.time() - t0
    eng = K.Engine(img, cfg)
    eng.set_graph(not args.no_graph)
    eng.set_mode(K.MODE_MULTI if args.mode == "multi" else K.MODE_PERSISTENT)
    persistent = eng.mode == K.MODE_PERSISTENT
    if args.mode == "persistent" and not persistent:
        print("bench.py: the persistent step does not fit this device; using --mode multi",
              file=sys.stderr)
    t_load = time.time() - t0 - t_img
    prompt = K.prompt_tokens(cfg)
    print(f"# {K.device_name(0)}; image {img.nbytes / 1e9:.2f} GB in {t_img:.1f} s, "
          f"upload {t_load:.1f} s", file=sys.stderr, flush=True)

    wall0 = time.perf_counter()
    toks, ms = eng.bench(prompt, args.warmup, steps)
    wall = time.perf_counter() - wall0
    tok_s = steps / (ms / 1e3)
    first_pos = P - 1 + args.warmup
    step_bytes = cfg.decode_bytes(first_pos, steps)
    gbps = step_bytes / (ms / 1e3) / 1e9
    print(f"# decode {steps} steps in {ms:.2f} ms ({tok_s:.1f} tok/s, {gbps:.0f} GB/s); "
          f"call wall {wall:.2f} s", file=sys.stderr, flush=True)

    # Per-launch durations: HIP events around every launch on the engine's
    # stream, over --profile-steps more decode steps continuing the run.
    prof_pos = first_pos + steps
    if prof_pos + args.profile_steps > cfg.seq_len:
        prof_pos = first_pos
    prof = eng.profile(int(toks[-1]), prof_pos, args.profile_steps)
    per_step_eager = sum(v[0] * v[1] for v in prof.values()) / args.profile_steps
    if persistent:
        # One launch is one decode step and the timed steps run back to back
        # on the engine's stream, so the kernel's average launch duration over
        # the timed region is the HIP-event time of that region per step (it
        # includes the few-microsecond gaps between launches); the algorithmic
        # bytes per launch are the timed positions' average.  The profile
        # steps' per-launch events are reported beside it.
        dom_name = "k_decode_persistent (whole decode step: every layer, classifier, argmax)"
        dom_ms = ms / steps
        dom_bytes = step_bytes / steps
        prof_bytes = cfg.decode_bytes(prof_pos, args.profile_steps) / args.profile_steps
    else:
        dom_name = "k_w13_swiglu (RMSNorm + W1/W3 GEMV + SwiGLU)"
        dom_ms = prof["w13"][0]
        dom_bytes = dominant_kernel_bytes(cfg)
    dom_gbps = dom_bytes / (dom_ms / 1e3) / 1e9
    traffic, traffic_src = measured_traffic("k_decode_persistent" if persistent else "k_w13_swiglu",
                                            cfg.name, "persistent" if persistent else "multi")
    print("# per-launch avg ms: " + ", ".join(f"{k} {v[0]:.4f} x{v[1]}" for k, v in prof.items() if v[1])
          + f"; step {per_step_eager:.3f} ms", file=sys.stderr, flush=True)

    # The box's own HBM rates (outside every timed region): a streaming read
    # of 2 GiB and a 1 GiB device copy, so the decode rate can be read
    # against what this device sustains as well as against the 8 TB/s spec.
    hbm = None
    if not args.no_hbm_probe:
        rd, cp = C.c_float(0.0), C.c_float(0.0)
        K.check(K.lib.kl_hbm_probe(1 << 30, 10, C.byref(rd), C.byref(cp)), "kl_hbm_probe")
        hbm = {"read_GBps": round(rd.value, 1), "copy_GBps": round(cp.value, 1),
               "probe": "kl_hbm_probe: 10 passes of a read of 2 GiB (one workgroup per CU, "
                        "16-byte loads over a contiguous chunk each) and of a 1 GiB "
                        "device-to-device copy (read + written bytes)"}
        print(f"# hbm probe {hbm}", file=sys.stderr, flush=True)

    del eng
    legs = {}
    prefill = None
    names = [] if args.configs == "none" else [c for c in args.configs.split(",") if c]
    for name in names:
        if name == cfg.name:
            continue
        reps = 3 if name == args.prefill_config else 1
        legs[name] = decode_leg(K, K.BASELINE[name], args.config_steps, args.config_warmup, reps)
        if name == args.prefill_config:
            prefill = legs[name]["prefill"]
    if args.prefill_config != "none" and prefill is None:
        prefill = measure_prefill(K, K.BASELINE[args.prefill_config])
    if prefill is not None:
        print(f"# prefill {prefill}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        # toks[j] is the token sampled at position P - 1 + j
        cpu = cpu_baseline(K, cfg, img, first_pos, steps, toks, args.cpu_seconds,
                           args.cpu_seconds_1t)
        print(f"# cpu baseline {cpu}", file=sys.stderr, flush=True)

    out = {
        "metric": METRIC,
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8w-f32" if cfg.quant else "f32",
        "data": "synthetic: seeded N(0,0.02) weights in the reference .bin layout, seeded "
                "uniform prompt ids",
        "config": {
            "workload": f"{cfg.name}: batch-1 greedy decode, {P}-token prompt then {steps} timed "
                        f"decode steps (positions {first_pos}..{first_pos + steps - 1})",
            "model": cfg.name,
            "global_batch": 1,
            "seq_len": cfg.seq_len,
            "parallelism": "single GPU",
            "mode": "persistent" if persistent else "multi",
            "graph": (not args.no_graph) and not persistent,
            "launch": ("cooperative" if os.environ.get("KL_PERSISTENT_LAUNCH") == "cooperative"
                       else "plain") if persistent else "stream",
        },
        "achieved_GBps": round(gbps, 1),
        "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "bytes_per_token": int(step_bytes / steps),
        "roofline": {
            "bound": "hbm",
            "kernel": dom_name,
            "achieved": round(dom_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dom_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "bytes_per_launch": int(dom_bytes),
            "avg_launch_ms": round(dom_ms, 5),
            "over": ("the timed region (HIP events around its back-to-back launches)" if persistent
                     else f"{args.profile_steps} profile steps (HIP events around each launch)"),
        },
        "launch_ms": {k: round(v[0], 5) for k, v in prof.items() if v[1]},
        "cpu_baseline": cpu,
    }
    if persistent:
        out["roofline"]["profile_steps"] = {
            "positions": f"{prof_pos}..{prof_pos + args.profile_steps - 1}",
            "avg_launch_ms": round(prof["step"][0], 5),
            "achieved": round(prof_bytes / (prof["step"][0] / 1e3) / 1e9, 1),
            "frac": round(prof_bytes / (prof["step"][0] / 1e3) / 1e9 / HBM_PEAK_GBPS, 4)}
    if hbm is not None:
        hbm["decode_frac_of_read"] = round(gbps / hbm["read_GBps"], 4)
        hbm["kernel_frac_of_read"] = round(dom_gbps / hbm["read_GBps"], 4)
        out["hbm_measured"] = hbm
    if prefill is not None:
        out["prefill"] = prefill
    if legs:
        out["configs"] = legs
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
