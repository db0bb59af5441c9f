#!/usr/bin/env python3
"""Benchmark of the PRIME moment-attention hot paths on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--decode-steps K2] [--no-cpu]

The headline is BASELINE.json's metric, "prefill tok/s + decode tok/s (B=256)
PRIME-125M": the PRIME-125M-shaped causal LM (12 layers, d_model 768, 12 x 64
heads, GELU MLP 3072, tied vocab 50304, bf16 weights, fp32 states, LayerNorm
QK-norm, random init).  One "step" is one prefill of B=32 x 2048 random token
ids (all layers, the states, and the last position's logits and greedy token);
W untimed steps, then K timed steps between synchronisations.
  value         prefill tokens/s = 32 * 2048 / (seconds per step)
  decode_tok_s  greedy decode tokens/s at B=256 (the metric's decode batch):
                the HIP-graph one-token step (embedding, 12 layers, lm_head,
                argmax), timed over --decode-steps steps after a 128-token
                prompt; decode_B32 (config 4's batch) rides along
  roofline      the prefill call against dense bf16 MFMA peak (algorithmic
                flops per call / measured seconds per call); decode_roofline
                the decode step against HBM peak (weights + state bytes per
                step / measured seconds per step)
  cpu_baseline  the fp32 PyTorch-CPU restatement of the same model
                (oracle/torch_cpu.py CausalLMCPU, the reference's chunked core
                with its O(Nc^2) carry) on the same weights: a bounded sample
                of the prefill, and decode steps at B=256 under
                decode_cpu_baseline
Extra keys carry the kernel-level workloads of BASELINE.json (run first; they
also bring the GPU clocks up before the headline):
  kernels.prefill_config2  the chunked prefill alone (B=8, H=12, L=8192), its
                fused chunk kernel's HBM roofline from HIP events inside the
                timed region, and the kernel's rocprof-calibrated traffic
  decode        the fused decode kernel at B=512 x 12 layers x 12 heads (and
                B=256), states pre-filled by 1024 tokens, HBM roofline
  delta, selective, hybrid, backward   the other built paths
  hbm_measured  achievable HBM bandwidth on this GPU
  gpu_clock     the graphics clock read before and after the headline
The CPU legs are the only use of oracle/ here, and only as timing baselines.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "prime-moment-attention_amd")]

PEAK_HBM = 8.0e12          # bytes/s, MI355X HBM3E
PEAK_BF16 = 2.5e15         # flop/s, dense bf16 MFMA
D = 64
STATE_BYTES = (2 * D * D + 3 * D + 1) * 4          # 33,540 B per (sequence, head)
PREFILL_BYTES_PER_TOKEN_HEAD = 3 * 2 * D + 2 * D   # bf16 q, k, v in + bf16 y out
PREFILL_FLOP_PER_TOKEN_HEAD = 6 * 64 * D + 8 * D * D  # intra 6CD + dS 4D^2 + carry readout 4D^2
DECODE_BYTES_PER_TILE = 2 * STATE_BYTES + 3 * 2 * D + 2 * D  # state r+w, bf16 q,k,v, bf16 y


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30, help="timed PRIME-125M prefill steps (B=32 x 2048 each)")
    ap.add_argument("--warmup", type=int, default=5, help="untimed prefill steps before them")
    ap.add_argument("--decode-steps", type=int, default=256, help="timed greedy decode steps of the model")
    ap.add_argument("--kernel-steps", type=int, default=200,
                    help="timed calls of each kernel-level leg (chunked prefill, selective, hybrid, backward)")
    ap.add_argument("--kernel-decode-steps", type=int, default=1000,
                    help="timed steps of the decode-kernel leg (12 layers each)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode legs")
    ap.add_argument("--no-model", action="store_true", help="skip the PRIME-125M model leg")
    ap.add_argument("--no-delta", action="store_true", help="skip the delta-rule (config 5) leg")
    ap.add_argument("--no-selective", action="store_true", help="skip the selective PRIME leg")
    ap.add_argument("--no-hybrid", action="store_true", help="skip the hybrid window-PRIME leg")
    ap.add_argument("--no-backward", action="store_true", help="skip the prefill-backward leg")
    ap.add_argument("--cpu-budget", type=float, default=6.0, help="seconds per CPU leg (approximate)")
    ap.add_argument("--detail", default=None,
                    help="write the full record here (default: gpurun_out/bench_full.json when that folder exists)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 1 GiB device copy 3 times (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    return ap.parse_args()


# ----------------------------------------------------------------- inputs
def qkv(shape, gen, device, dtype):
    """q, k, v ~ N(0,1); q and k L2-normalised over D, rounded to dtype, q / 8."""
    import torch
    out = []
    for i in range(3):
        x = torch.randn(*shape, generator=gen, device=device, dtype=torch.float32)
        if i < 2:
            x = x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        x = x.to(dtype)
        if i == 0:
            x = x / 8
        out.append(x)
    return out


def timed(fn, steps, warmup):
    """W untimed calls, then K calls bracketed by synchronisation; ms per call
    from events on the current stream (the stream the library launches on)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def kernel_ms(lib, kid):
    ms, n = lib.timer_read(kid)
    return (ms / n if n else None), n


def load_traffic():
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by the same counter's reading for a
    copy kernel of known size); None if that summary is absent."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


# ----------------------------------------------------------------- HBM probe
def bench_hbm(lib, torch, dev):
    """Achievable HBM bandwidth on this GPU, for the fractions against the
    measured rather than the published peak: the library's nontemporal
    16-byte stream kernel (prime_hbm_stream) copying 1 GiB (read + write) and
    reading 2.5 GB once (both beyond the 256 MB Infinity Cache), the best of
    a sweep over grid sizes."""
    def tm(fn, reps=10):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps * 1e-3
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    n = 1 << 30
    src = torch.ones(n // 4, device=dev)
    dst = torch.empty_like(src)
    copy = {b: 2 * n / tm(lambda: lib.hbm_stream(src, dst, True, b)) for b in (2 * cus, 4 * cus, 8 * cus, 16 * cus)}
    del src, dst
    m = 5 * (1 << 29)  # 2.5 GiB
    big = torch.ones(m // 4, device=dev)
    sink = torch.empty(16 * cus * 16 // 4, device=dev)
    read = {b: m / tm(lambda: lib.hbm_stream(big, sink, False, b)) for b in (2 * cus, 4 * cus, 8 * cus, 16 * cus)}
    del big, sink
    torch.cuda.empty_cache()
    cb, rb = max(copy.values()), max(read.values())
    return {"copy_GBps": cb / 1e9, "read_GBps": rb / 1e9, "achievable_GBps": max(cb, rb) / 1e9,
            "method": "prime_hbm_stream: nontemporal 16-byte copy of 1 GiB (read + write) and read of 2.5 GiB, "
                      "best over 2-16 workgroups per CU"}


# ----------------------------------------------------------------- prefill
def bench_prefill(args, lib, torch, dev):
    B, H, L, C = 8, 12, 8192, 64
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    q, k, v = qkv((B, H, L, D), gen, dev, torch.bfloat16)
    lam = torch.empty(H, device=dev).uniform_(0.99, 0.9999, generator=gen)
    y = torch.empty(B, H, L, D, device=dev, dtype=torch.bfloat16)
    st = lib.new_state(B, H, D, dev)
    step = lib.bind_chunked_prefill(q, k, v, lam, 1.0, C, None, y, st)
    ws = step.buffers[7]
    for _ in range(50):
        step()
    torch.cuda.synchronize()
    # the call alone, no instrumentation
    ms = timed(step, args.kernel_steps, 0)
    # the same steps again with every kernel of the call bracketed by HIP events
    # on the call's stream, for the per-kernel durations (an event pair around
    # the dominant kernel alone would open while the preceding scan kernel still
    # runs and count part of it); the events add a few microseconds per call
    ids = (lib.KERNEL_PREFILL_CHUNKS, lib.KERNEL_PREFILL_SEGMENTS, lib.KERNEL_SEGMENT_SCAN)
    lib.timer_reset()
    lib.timer_enable(*ids)
    ms_events = timed(step, args.kernel_steps, 0)
    lib.timer_enable()
    kern = {lib.KERNEL_NAMES[kid]: kernel_ms(lib, kid) for kid in ids}
    main_ms, main_n = kernel_ms(lib, lib.KERNEL_PREFILL_CHUNKS)
    lib.timer_reset()
    ok = bool(torch.isfinite(y).all().item())
    tokens = B * L
    algo_bytes = B * H * L * PREFILL_BYTES_PER_TOKEN_HEAD + B * H * STATE_BYTES
    flops = B * H * L * PREFILL_FLOP_PER_TOKEN_HEAD
    return dict(B=B, H=H, L=L, C=C, ms=ms, tokens=tokens, bytes=algo_bytes, flops=flops, finite=ok,
                kernels={n: {"avg_us": None if t is None else t * 1e3, "launches": c} for n, (t, c) in kern.items()},
                ms_events=ms_events, main_ms=main_ms, main_n=main_n, ws_bytes=0 if ws is None else ws.numel())


# ----------------------------------------------------------------- decode
def bench_decode(args, lib, torch, dev, B, layers=12, H=12, pool=16, prefill_tokens=1024):
    gen = torch.Generator(device=dev).manual_seed(args.seed + 1000 + B)
    lams = [torch.empty(H, device=dev).uniform_(0.99, 0.9999, generator=gen) for _ in range(layers)]
    states = [lib.new_state(B, H, D, dev) for _ in range(layers)]
    # states pre-filled by the library's own prefill of 1024 random tokens
    chunkB = max(1, min(B, 128))
    for l in range(layers):
        for b0 in range(0, B, chunkB):
            nb = min(chunkB, B - b0)
            q, k, v = qkv((nb, H, prefill_tokens, D), gen, dev, torch.bfloat16)
            yp = torch.empty_like(q)
            part = tuple(t[b0:b0 + nb] for t in states[l])
            lib.chunked_prefill(q, k, v, lams[l], 1.0, 64, None, yp, part)
        del q, k, v, yp
    torch.cuda.synchronize()
    toks = [[qkv((B, H, D), gen, dev, torch.bfloat16) for _ in range(pool)] for _ in range(layers)]
    ys = [torch.empty(B, H, D, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    calls = [[lib.bind_decode_step(*toks[l][p], lams[l], 1.0, states[l], states[l], ys[l])
              for l in range(layers)] for p in range(pool)]
    it = [0]

    def step():
        for c in calls[it[0] % pool]:
            c()
        it[0] += 1
    steps = args.kernel_decode_steps
    # a step is `layers` back-to-back launches of the decode kernel and nothing
    # else, so the events around the timed region give the launch duration
    # (ms per step / layers, gaps between launches included) without events
    # between the launches
    ms = timed(step, steps, 20)
    kms, n = ms / layers, steps * layers
    ok = all(bool(torch.isfinite(y).all().item()) for y in ys)
    per_launch = B * H * DECODE_BYTES_PER_TILE
    achieved = per_launch / (kms * 1e-3)
    return {
        "workload": f"decode step B={B} x {layers} layers x {H} heads, D=64, bf16 q/k/v, fp32 state in place, "
                    f"bf16 y; states pre-filled by {prefill_tokens} tokens; one launch per layer",
        "tok_s": B / (ms * 1e-3), "ms_per_step": ms, "steps": steps, "finite": ok,
        "state_bytes": layers * B * H * STATE_BYTES,
        "roofline": {"kernel": "decode_step_kernel", "bound": "hbm", "achieved": achieved / 1e9,
                     "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": achieved / PEAK_HBM,
                     "bytes_per_launch": per_launch, "avg_launch_us": kms * 1e3, "launches": n,
                     "traffic": None},
    }


# ----------------------------------------------------------------- model
MODEL_B, MODEL_L, DECODE_B, DECODE_PROMPT = 32, 2048, 256, 128


def model_flop_per_token(cfg):
    """Algorithmic flops per prefill token: 2 x (q, k, v, o: 4 d^2; up and
    down: 2 d f) per layer, plus the chunked attention's 57,344 flop per
    token-head.  The lm_head runs for the last position only: greedy decoding
    needs no other logits."""
    d, f, nl, H = cfg.hidden_size, cfg.intermediate_size, cfg.num_layers, cfg.num_heads
    return 2 * nl * (4 * d * d + 2 * d * f) + nl * H * PREFILL_FLOP_PER_TOKEN_HEAD


def model_decode_bytes_per_step(cfg, B):
    """Algorithmic HBM bytes of one greedy step: every bf16 weight read once
    (the 12 layers' projections and MLP, and the tied 50304 x 768 lm_head),
    and every fp32 state read and written once."""
    d, f, nl, H, V = cfg.hidden_size, cfg.intermediate_size, cfg.num_layers, cfg.num_heads, cfg.vocab_size
    weights = 2 * (nl * (4 * d * d + 2 * d * f) + V * d)
    return weights + 2 * nl * B * H * STATE_BYTES


def bench_model(args, lib, torch, dev):
    """The headline: PRIME-125M-shaped causal LM (12 layers, d_model 768,
    12 x 64 heads, GELU MLP 3072, tied 50304 vocab, bf16 weights, fp32 states,
    LayerNorm QK-norm), random init.  One step = the prefill of B=32 x 2048
    random ids: the 12 layers with their final states, the last position's
    logits and its greedy token (model.forward + argmax).  Then greedy decode
    with the HIP-graph step at B=256 (a 128-token prompt; the step's cost does
    not depend on the position) and at B=32 after the 2048-token prefill."""
    from prime_moment_attention import GreedyDecoder, PrimeForCausalLM, prime_125m_config
    cfg = prime_125m_config("gelu")
    torch.manual_seed(args.seed)
    model = PrimeForCausalLM(cfg).to(device=dev, dtype=torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(args.seed + 7)
    V = cfg.vocab_size
    ids = torch.randint(0, V, (MODEL_B, MODEL_L), device=dev, generator=gen)
    tok = torch.empty(MODEL_B, 1, dtype=torch.int64, device=dev)

    def prefill():
        with torch.no_grad():
            out = model(ids, return_states=True, logits_to_keep=1)
            lib.argmax(out["logits"][:, -1, :], tok)
        return out

    clock_before = read_gpu_clock()
    for _ in range(args.warmup):
        prefill()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        prefill()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    clock_after = read_gpu_clock()
    # the attention kernels of the same steps, stamped by their dispatches
    ids_k = (lib.KERNEL_PREFILL_CHUNKS, lib.KERNEL_PREFILL_SEGMENTS, lib.KERNEL_SEGMENT_SCAN)
    lib.timer_reset()
    lib.timer_enable(*ids_k)
    nk = min(args.steps, 10)
    for _ in range(nk):
        prefill()
    torch.cuda.synchronize()
    lib.timer_enable()
    kern = {lib.KERNEL_NAMES[kid]: kernel_ms(lib, kid) for kid in ids_k}
    lib.timer_reset()
    attn_us = {n: {"avg_us": None if t is None else t * 1e3, "launches_per_step": c / nk}
               for n, (t, c) in kern.items() if c}
    fused_ms = kern[lib.KERNEL_NAMES[lib.KERNEL_PREFILL_CHUNKS]][0]
    attn_per_layer_us = sum(v["avg_us"] * v["launches_per_step"] for v in attn_us.values()) / cfg.num_layers
    th = MODEL_B * cfg.num_heads * MODEL_L
    attn_bytes = th * PREFILL_BYTES_PER_TOKEN_HEAD + MODEL_B * cfg.num_heads * STATE_BYTES
    tokens = MODEL_B * MODEL_L
    flops = tokens * model_flop_per_token(cfg)
    out = {"prefill": {"B": MODEL_B, "L": MODEL_L, "ms": ms, "tok_s": tokens / (ms * 1e-3),
                       "flop_per_token": model_flop_per_token(cfg), "flop_per_step": flops,
                       "attention_kernels": attn_us, "attention_us_per_layer": attn_per_layer_us,
                       "attention_roofline": {
                           "kernel": "prefill_bf16_kernel (fused chunk loop, QK-norm on load) per layer",
                           "bound": "hbm", "bytes_per_launch": attn_bytes, "avg_launch_us": fused_ms * 1e3,
                           "achieved": attn_bytes / (fused_ms * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                           "frac": attn_bytes / (fused_ms * 1e-3) / PEAK_HBM}},
           "params": sum(p.numel() for p in model.parameters()),
           "gpu_clock": {"before_prefill": clock_before, "after_prefill": clock_after}}
    out["roofline"] = {"kernel": "PRIME-125M prefill step, all kernels (library GEMMs of the projections and MLP, "
                                 "the fused PRIME prefill, norms, GELU)", "bound": "mfma",
                       "achieved": flops / (ms * 1e-3) / 1e12, "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                       "frac": flops / (ms * 1e-3) / PEAK_BF16, "traffic": None,
                       "flop_per_step": flops, "avg_step_ms": ms}

    def decode_leg(Bd, prompt):
        dec = GreedyDecoder(model, use_graph=True)
        dec.prefill(prompt)
        for _ in range(4):
            dec.step()  # the first step captures the graph
        torch.cuda.synchronize()
        s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_.record()
        for _ in range(args.decode_steps):
            dec.step()
        e_.record()
        torch.cuda.synchronize()
        dms = s_.elapsed_time(e_) / args.decode_steps
        byts = model_decode_bytes_per_step(cfg, Bd)
        res = {"B": Bd, "prompt_tokens": prompt.shape[1], "steps": args.decode_steps, "ms_per_step": dms,
               "tok_s": Bd / (dms * 1e-3),
               "roofline": {"kernel": f"greedy decode step at B={Bd}, all kernels (HIP graph)", "bound": "hbm",
                            "achieved": byts / (dms * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                            "frac": byts / (dms * 1e-3) / PEAK_HBM, "traffic": None, "bytes_per_step": byts,
                            "avg_step_ms": dms},
               "states": dec.states}
        del dec
        return res

    d256 = decode_leg(DECODE_B, torch.randint(0, V, (DECODE_B, DECODE_PROMPT), device=dev, generator=gen))
    d32 = decode_leg(MODEL_B, ids)
    out["decode_B256"] = {k: v for k, v in d256.items() if k != "states"}
    out["decode_B32"] = {k: v for k, v in d32.items() if k != "states"}
    out["_model"], out["_ids"] = model, ids
    out["_decode_states_B256"] = d256["states"]
    torch.cuda.empty_cache()
    return out


def bench_model_selective(args, torch, dev):
    """The same model with the selective attention of the shipped PRIME-125M
    (per-token decays, beta-weighted keys; off the identity initialisation):
    prefill B=32 x 2048 and greedy decode at B=256."""
    from prime_moment_attention import GreedyDecoder, PrimeForCausalLM, prime_125m_config
    torch.manual_seed(args.seed)
    model = PrimeForCausalLM(prime_125m_config("gelu", use_selective=True)).to(
        device=dev, dtype=torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(args.seed + 7)
    with torch.no_grad():
        for layer in model.layers:
            layer.self_attn.delta_proj.weight.normal_(0.0, 0.01, generator=gen)
            layer.self_attn.log_beta.uniform_(-0.5, 0.5, generator=gen)
    V = model.config.vocab_size
    ids = torch.randint(0, V, (MODEL_B, MODEL_L), device=dev, generator=gen)
    run = lambda: model(ids, return_states=True, logits_to_keep=1)
    with torch.no_grad():
        ms = timed(run, 5, 2)
    dec = GreedyDecoder(model, use_graph=True)
    dec.prefill(torch.randint(0, V, (DECODE_B, DECODE_PROMPT), device=dev, generator=gen))
    dms = timed(dec.step, max(64, args.decode_steps // 2), 4)
    del model, dec
    torch.cuda.empty_cache()
    return {"workload": "PRIME-125M shape with selective attention (per-token decays, beta-weighted keys): "
                        "prefill B=32 x 2048, greedy decode B=256",
            "prefill": {"ms": ms, "tok_s": MODEL_B * MODEL_L / (ms * 1e-3)},
            "decode_B256": {"ms_per_step": dms, "tok_s": DECODE_B / (dms * 1e-3)}}


def read_gpu_clock():
    """The graphics clock(s) of the visible GPU in MHz, from amd-smi (or
    rocm-smi); an error string when neither answers.  Under a profiler no tool
    is spawned (their launch scripts re-exec an interpreter, which the
    profiler's preloaded library sees as a program replacing itself): the
    starred levels of the driver's sysfs ``pp_dpm_sclk`` tables are read
    instead, for every card the host shows."""
    import glob
    import subprocess
    if "rocprof" in os.environ.get("LD_PRELOAD", "") or any(k.startswith("ROCPROF") for k in os.environ):
        levels = {}
        for f in sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")):
            try:
                lines = [ln for ln in open(f).read().splitlines() if ":" in ln]
            except OSError:
                continue
            mhz = [int("".join(ch for ch in ln.split(":")[1] if ch.isdigit()) or 0) for ln in lines]
            cur = [m for m, ln in zip(mhz, lines) if ln.rstrip().endswith("*")]
            if mhz:
                levels[f.split("/")[4]] = {"cur_mhz": cur[0] if cur else None, "max_mhz": max(mhz)}
        return {"tool": "sysfs pp_dpm_sclk", "cards": levels} if levels else {"error": "not read under a profiler"}
    err = "no clock source"
    for cmd in (["amd-smi", "metric", "--clock", "--json"], ["rocm-smi", "--showclocks", "--json"]):
        try:
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=20)
        except (OSError, subprocess.TimeoutExpired) as exc:
            err = f"{cmd[0]}: {exc}"
            continue
        try:
            data = json.loads(r.stdout[r.stdout.find("[") if r.stdout.lstrip().startswith("[") else
                                      r.stdout.find("{"):])
        except ValueError:
            err = f"{cmd[0]}: unparsed output {r.stdout[:120]!r}"
            continue
        found = {}

        def walk(x, path):
            if isinstance(x, dict):
                for k, v in x.items():
                    walk(v, path + (str(k),))
            elif isinstance(x, list):
                for i, v in enumerate(x):
                    walk(v, path + (str(i),))
            else:
                p = "/".join(path).lower()
                if ("gfx" in p or "sclk" in p) and ("clk" in p or "value" in p or "clock" in p):
                    found["/".join(path)] = x
        walk(data, ())
        cur = {k.split("/")[-3]: v for k, v in found.items() if k.endswith("/clk/value")}
        mx = [v for k, v in found.items() if k.endswith("/max_clk/value")]
        if cur:
            return {"tool": cmd[0], "gfx_mhz": cur, "max_mhz": mx[0] if mx else None}
        if found:
            return {"tool": cmd[0], "raw": dict(list(found.items())[:8])}
        err = f"{cmd[0]}: no graphics clock in its output"
    return {"error": err}


# ----------------------------------------------------------------- selective
def bench_selective(args, lib, torch, dev):
    """Selective PRIME (selective.py:264-444) at the chunked-prefill shape
    (B=8, H=12, L=8192, bf16 q/k/v as config 2) with per-token decays
    lambda_t = exp(-softplus(N(0,1)) / tau_h), tau_h ~ U[8, 2000], beta_h ~
    U[0.5, 2]; then the decode step at B=256 x 12 layers (one launch per layer,
    replayed from a HIP graph)."""
    B, H, L = 8, 12, 8192
    gen = torch.Generator(device=dev).manual_seed(args.seed + 11)
    q, k, v = qkv((B, H, L, D), gen, dev, torch.bfloat16)
    tau = torch.empty(H, device=dev).uniform_(8.0, 2000.0, generator=gen)
    beta = torch.empty(H, device=dev).uniform_(0.5, 2.0, generator=gen)
    delta = torch.nn.functional.softplus(torch.randn(B, H, L, device=dev, generator=gen))
    log_decay = (-delta / tau.view(1, H, 1)).contiguous()
    y = torch.empty(B, H, L, D, device=dev, dtype=torch.bfloat16)
    st = lib.new_state(B, H, D, dev)
    ws = torch.empty(lib.workspace_size(B, H, L), dtype=torch.uint8, device=dev)
    run = lambda: lib.selective_prefill(q, k, v, log_decay, beta, 1.0, None, y, st, workspace=ws)
    ids = (lib.KERNEL_PREFILL_CHUNKS, lib.KERNEL_PREFILL_SEGMENTS, lib.KERNEL_SEGMENT_SCAN)
    for _ in range(20):
        run()
    torch.cuda.synchronize()
    lib.timer_reset()
    lib.timer_enable(*ids)
    steps = max(50, args.kernel_steps // 4)
    ms = timed(run, steps, 0)
    lib.timer_enable()
    kern = {lib.KERNEL_NAMES[kid]: kernel_ms(lib, kid) for kid in ids}
    lib.timer_reset()
    main_ms = kern[lib.KERNEL_NAMES[lib.KERNEL_PREFILL_CHUNKS]][0]
    # q, k, v, y bf16 and the fp32 log decay per token-head, plus the final state
    algo = B * H * L * (PREFILL_BYTES_PER_TOKEN_HEAD + 4) + B * H * STATE_BYTES
    out = {"workload": "selective PRIME prefill, B=8 x H=12 x L=8192, D=64, bf16 q/k/v, per-token decays, "
                       "beta-weighted keys, zero initial state, bf16 y, fp32 final state",
           "prefill": {"tok_s": B * L / (ms * 1e-3), "ms": ms, "finite": bool(torch.isfinite(y).all().item()),
                       "kernels": {n: {"avg_us": None if t is None else t * 1e3, "launches": c}
                                   for n, (t, c) in kern.items()},
                       "roofline": {"kernel": "prefill_bf16_kernel<false, true, true, true, false>", "bound": "hbm",
                                    "bytes_per_launch": algo, "avg_launch_us": main_ms * 1e3,
                                    "achieved": algo / (main_ms * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9,
                                    "unit": "GB/s", "frac": algo / (main_ms * 1e-3) / PEAK_HBM}}}
    # the same with fp32 q/k/v and y (the fp32 kernel; segments for few long sequences)
    q32, k32, v32 = (t.float() for t in (q, k, v))
    y32 = torch.empty(B, H, L, D, device=dev, dtype=torch.float32)
    run32 = lambda: lib.selective_prefill(q32, k32, v32, log_decay, beta, 1.0, None, y32, st, workspace=ws)
    for _ in range(3):
        run32()
    torch.cuda.synchronize()
    ms32 = timed(run32, max(10, args.kernel_steps // 20), 0)
    out["prefill_f32"] = {"tok_s": B * L / (ms32 * 1e-3), "ms": ms32,
                          "finite": bool(torch.isfinite(y32).all().item())}
    del q, k, v, y, delta, log_decay, ws, q32, k32, v32, y32
    # decode B=256 x 12 layers
    Bd, layers = 256, 12
    states = []
    for _ in range(layers):
        s_ = lib.new_state(Bd, H, D, dev, zero=True)
        for t in s_:
            t.normal_(generator=gen).mul_(0.1)
        s_[3].abs_().add_(1.0)
        states.append(s_)
    toks = [qkv((Bd, H, D), gen, dev, torch.bfloat16) for _ in range(layers)]
    lams = [torch.exp(-torch.nn.functional.softplus(torch.randn(Bd, H, device=dev, generator=gen)) / tau.view(1, H))
            .contiguous() for _ in range(layers)]
    ys = [torch.empty(Bd, H, D, device=dev, dtype=torch.bfloat16) for _ in range(layers)]
    gates = [lib.selective_gate(Bd, H, decay_bh=lam) for lam in lams]

    def step():
        for l in range(layers):
            lib.selective_decode_step(*toks[l], gates[l], beta, 1.0, None, states[l], states[l], ys[l])
    s0 = torch.cuda.Stream()
    s0.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s0):
        step()
    torch.cuda.current_stream().wait_stream(s0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    dsteps = max(100, args.kernel_decode_steps // 4)
    dms = timed(g.replay, dsteps, 10)
    per_launch = Bd * H * (DECODE_BYTES_PER_TILE + 4)
    out["decode_B256"] = {"tok_s": Bd / (dms * 1e-3), "ms_per_step": dms, "steps": dsteps,
                          "finite": all(bool(torch.isfinite(t).all().item()) for t in ys),
                          "roofline": {"kernel": "decode_step_kernel (selective)", "bound": "hbm",
                                       "bytes_per_launch": per_launch, "avg_launch_us": dms / layers * 1e3,
                                       "achieved": per_launch / (dms / layers * 1e-3) / 1e9,
                                       "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                                       "frac": per_launch / (dms / layers * 1e-3) / PEAK_HBM}}
    del g, states
    torch.cuda.empty_cache()
    return out


# ----------------------------------------------------------------- delta rule
def bench_hybrid(args, lib, torch, dev):
    """The hybrid window-PRIME pieces (prime_cpp_kernel.cpp:6-117 replaced by
    prime_chunked_prefill at eps 1e-3, prime_accumulate, prime_decode_update,
    prime_decode_readout): the eviction accumulator over B=8 x H=12 x L=8192
    bf16 k/v, the fp32-input prefill (the reference's hybrid casts q/k/v to
    fp32, hybrid.py:109-114) at the same shape, and the per-token update and
    readout at B=256 x 12 layers (HIP-graph replays)."""
    B, H, L = 8, 12, 8192
    gen = torch.Generator(device=dev).manual_seed(args.seed + 13)
    q, k, v = qkv((B, H, L, D), gen, dev, torch.bfloat16)
    lam = torch.empty(H, device=dev).uniform_(0.99, 0.9999, generator=gen)
    st = lib.new_state(B, H, D, dev)
    ws = torch.empty(lib.accumulate_workspace_size(B, H, L), dtype=torch.uint8, device=dev)
    out = {}

    def leg(run, ids, main_id, algo, steps, tokens, workload, kernel, names=None):
        names = names or lib.KERNEL_NAMES
        for _ in range(10):
            run()
        torch.cuda.synchronize()
        lib.timer_reset()
        lib.timer_enable(*ids)
        ms = timed(run, steps, 0)
        lib.timer_enable()
        kern = {names[kid]: kernel_ms(lib, kid) for kid in ids}
        lib.timer_reset()
        main_ms = kern[names[main_id]][0]
        return {"workload": workload, "tok_s": tokens / (ms * 1e-3), "ms": ms,
                "kernels": {n: {"avg_us": None if t is None else t * 1e3, "launches": c} for n, (t, c) in kern.items()},
                "roofline": {"kernel": kernel, "bound": "hbm", "bytes_per_launch": algo,
                             "avg_launch_us": main_ms * 1e3, "achieved": algo / (main_ms * 1e-3) / 1e9,
                             "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": algo / (main_ms * 1e-3) / PEAK_HBM}}

    steps = max(50, args.kernel_steps // 4)
    # bf16 k, v in; fp32 final state out
    out["accumulate"] = leg(lambda: lib.accumulate(k, v, lam, None, st, workspace=ws),
                            (lib.KERNEL_PREFILL_SEGMENTS, lib.KERNEL_SEGMENT_SCAN), lib.KERNEL_PREFILL_SEGMENTS,
                            B * H * L * 4 * D + B * H * STATE_BYTES, steps, B * L,
                            "prime_accumulate, B=8 x H=12 x L=8192 bf16 k/v, zero initial state",
                            "prefill_bf16_kernel<true, false, false, false, false> (state-only)")
    del q, k, v
    q32, k32, v32 = qkv((B, H, L, D), gen, dev, torch.float32)
    y32 = torch.empty(B, H, L, D, device=dev)
    ws2 = torch.empty(lib.workspace_size(B, H, L), dtype=torch.uint8, device=dev)
    ids = (lib.KERNEL_PREFILL_CHUNKS, lib.KERNEL_PREFILL_SEGMENTS, lib.KERNEL_SEGMENT_SCAN)
    out["prefill_f32"] = leg(lambda: lib.chunked_prefill(q32, k32, v32, lam, 1e-3, 64, None, y32, st, workspace=ws2),
                             ids, lib.KERNEL_PREFILL_CHUNKS, B * H * L * 16 * D + B * H * STATE_BYTES,
                             max(20, steps // 2), B * L,
                             "prime_chunked_prefill with fp32 q/k/v/y and eps 1e-3 (prime_prefill_cpp), "
                             "B=8 x H=12 x L=8192", "prefill_kernel<true, false> (fp32 inputs)",
                             {lib.KERNEL_PREFILL_CHUNKS: "prefill_kernel<true, false>",
                              lib.KERNEL_PREFILL_SEGMENTS: "prefill_kernel<true, true>",
                              lib.KERNEL_SEGMENT_SCAN: "segment_scan_kernel"})
    del q32, k32, v32, y32, ws, ws2
    # per-token update and readout, B=256 x 12 layers
    Bd, layers = 256, 12
    states = []
    for _ in range(layers):
        s_ = lib.new_state(Bd, H, D, dev, zero=True)
        for t in s_:
            t.normal_(generator=gen).mul_(0.1)
        s_[3].abs_().add_(1.0)
        states.append(s_)
    toks = [qkv((Bd, H, D), gen, dev, torch.float32) for _ in range(layers)]
    ys = [torch.empty(Bd, H, D, device=dev) for _ in range(layers)]
    for name, fn, per_tile in (
            ("update_B256", lambda l: lib.decode_update(toks[l][1], toks[l][2], lam, states[l], states[l]),
             2 * STATE_BYTES + 2 * 4 * D),
            ("readout_B256", lambda l: lib.decode_readout(toks[l][0], 1e-3, states[l], ys[l]),
             STATE_BYTES + 2 * 4 * D)):
        def step():
            for l in range(layers):
                fn(l)
        s0 = torch.cuda.Stream()
        s0.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s0):
            step()
        torch.cuda.current_stream().wait_stream(s0)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        dsteps = max(100, args.kernel_decode_steps // 4)
        dms = timed(g.replay, dsteps, 10)
        per_launch = Bd * H * per_tile
        out[name] = {"tok_s": Bd / (dms * 1e-3), "ms_per_step": dms, "steps": dsteps, "layers": layers,
                     "roofline": {"kernel": "decode_step_kernel (" + name.split("_")[0] + " only)", "bound": "hbm",
                                  "bytes_per_launch": per_launch, "avg_launch_us": dms / layers * 1e3,
                                  "achieved": per_launch / (dms / layers * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9,
                                  "unit": "GB/s", "frac": per_launch / (dms / layers * 1e-3) / PEAK_HBM}}
        del g
    del states
    torch.cuda.empty_cache()
    return out


BWD_FLOP_PER_TOKEN_HEAD = 2 * 2 * 64 * 64 * 768 // 64  # two passes, 7 GEMM blocks each: 196,608 flop


def bench_backward(args, lib, torch, dev):
    """Backward of the chunked prefill (prime_chunked_prefill_backward): dq pass
    + dk/dv pass, bf16 q/k/v/dy, fp32 gradients, zero initial state, at the
    config-2 shape (B=8 x H=12 x L=8192) and at a training shape (B=32 x
    H=12 x L=2048).  Algorithmic bytes per token-head: q, k, v, dy read by both
    passes (2 x 512 B), dq, dk, dv written (3 x 256 B fp32), 16 B of per-token
    denominators; flop per token-head: 196,608 (MFMA blocks of both passes).
    The config-2 shape once more with fp32 q/k/v/dy (the fp32 passes; bytes
    counted as for bf16, so its fraction is a lower bound)."""
    out = {}
    for (B, H, L, dt) in ((8, 12, 8192, torch.bfloat16), (32, 12, 2048, torch.bfloat16),
                          (8, 12, 8192, torch.float32)):
        gen = torch.Generator(device=dev).manual_seed(args.seed + 17 + B)
        q, k, v = qkv((B, H, L, D), gen, dev, dt)
        dy = torch.randn(B, H, L, D, device=dev, generator=gen).to(dt)
        lam = torch.empty(H, device=dev).uniform_(0.99, 0.9999, generator=gen)
        g = [torch.empty(B, H, L, D, device=dev) for _ in range(3)]
        ws = torch.empty(lib.backward_workspace_size(B, H, L), dtype=torch.uint8, device=dev)
        run = lambda: lib.chunked_prefill_backward(q, k, v, lam, 1.0, None, dy, None, *g, None, workspace=ws)
        ids = (lib.KERNEL_PREFILL_SEGMENTS, lib.KERNEL_SEGMENT_SCAN, lib.KERNEL_BWD_DQ, lib.KERNEL_BWD_DUAL,
               lib.KERNEL_BWD_DUAL_SCAN, lib.KERNEL_BWD_DKV)
        for _ in range(5):
            run()
        torch.cuda.synchronize()
        lib.timer_reset()
        lib.timer_enable(*ids)
        steps = max(10, args.kernel_steps // 20)
        ms = timed(run, steps, 0)
        lib.timer_enable()
        kern = {lib.KERNEL_NAMES[kid]: kernel_ms(lib, kid) for kid in ids}
        lib.timer_reset()
        th = B * H * L
        byts = th * (2 * 512 + 3 * 256 + 16)
        flops = th * BWD_FLOP_PER_TOKEN_HEAD
        kern = {n: v for n, v in kern.items() if v[1]}  # the segment kernels run only for few long sequences
        kt = sum(t for t, _ in kern.values())
        out[f"B{B}_H{H}_L{L}" + ("_f32" if dt == torch.float32 else "")] = {
            "tok_s": B * L / (ms * 1e-3), "ms": ms,
            "finite": all(bool(torch.isfinite(t).all().item()) for t in g),
            "kernels": {n: {"avg_us": None if t is None else t * 1e3, "launches": c} for n, (t, c) in kern.items()},
            "roofline": {"bound": "hbm", "bytes_per_call": byts, "flop_per_call": flops,
                         "kernels_us": kt * 1e3, "achieved_GBps": byts / (kt * 1e-3) / 1e9,
                         "hbm_frac": byts / (kt * 1e-3) / PEAK_HBM,
                         "tflops": flops / (kt * 1e-3) / 1e12, "mfma_frac": flops / (kt * 1e-3) / PEAK_BF16}}
        del q, k, v, dy, g, ws
        torch.cuda.empty_cache()
    return out


def bench_delta(args, lib, torch, dev):
    """Chunked gated delta-rule prefill: B=1, H=12, D=64,
    L=131072, chunk 64, bf16 q/k/v (N(0,1), QK-normed, q / 8), beta ~
    sigmoid(N(0,1)), alpha = per-head lambda ~ U[0.99, 0.9999], Lyapunov bound
    25.  Whole-sequence tok/s, then the sequence again in 16384-token pieces
    carrying the state, each piece timed, with the device memory in use after
    each piece (flat state memory, sustained throughput)."""
    B, H, L = 1, 12, 131072
    gen = torch.Generator(device=dev).manual_seed(args.seed + 5)
    q, k, v = qkv((B, H, L, D), gen, dev, torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, H, L, device=dev, generator=gen)).contiguous()
    lam = torch.empty(H, device=dev).uniform_(0.99, 0.9999, generator=gen)
    alpha = lam.view(1, H, 1).expand(B, H, L).contiguous()
    y = torch.empty(B, H, L, D, device=dev, dtype=torch.bfloat16)
    st = torch.empty(B, H, D, 2 * D, device=dev)
    ws = torch.empty(lib.delta_workspace_size(B, H, L), dtype=torch.uint8, device=dev)
    run = lambda: lib.delta_prefill(q, k, v, beta, alpha, 0.9995, 1e-5, 25.0, None, y, st, workspace=ws)
    run()
    torch.cuda.synchronize()
    reps = 3
    # the whole-sequence time without the library's kernel timer (its events
    # add a record per launch), then a second pass for the per-kernel averages
    ms = timed(run, reps, 0)
    lib.timer_reset()
    lib.timer_enable(lib.KERNEL_DELTA_PREP, lib.KERNEL_DELTA_SCAN)
    timed(run, reps, 0)
    lib.timer_enable()
    kern = {lib.KERNEL_NAMES[kid]: kernel_ms(lib, kid) for kid in (lib.KERNEL_DELTA_PREP, lib.KERNEL_DELTA_SCAN)}
    lib.timer_reset()
    ok = bool(torch.isfinite(y).all().item())
    nrm = float(st.norm(dim=(2, 3)).max().item())
    # pieces of 16384 tokens, state carried in place
    P = 16384
    pieces = []
    sp = torch.zeros(B, H, D, 2 * D, device=dev)
    ws_p = torch.empty(lib.delta_workspace_size(B, H, P), dtype=torch.uint8, device=dev)
    for i in range(L // P):
        sl = slice(i * P, (i + 1) * P)
        piece = lambda: lib.delta_prefill(q[:, :, sl], k[:, :, sl], v[:, :, sl], beta[:, :, sl].contiguous(),
                                          alpha[:, :, sl].contiguous(), 0.9995, 1e-5, 25.0, sp, y[:, :, sl], sp,
                                          workspace=ws_p)
        t = timed(piece, 1, 0)
        pieces.append({"tokens_end": (i + 1) * P, "tok_s": P / (t * 1e-3),
                       "mem_allocated_MB": torch.cuda.memory_allocated(dev) / 1e6})
    flops = B * H * L * (11 * 64 * D + 12 * D * D)
    return {"workload": "chunked delta-rule prefill, BASELINE config 5: B=1 x H=12 x L=131072, D=64, chunk 64, "
                        "bf16 q/k/v, beta ~ sigmoid(N(0,1)), alpha = per-head lambda U[0.99,0.9999], bound 25",
            "tok_s": B * L / (ms * 1e-3), "ms": ms, "finite": ok, "state_norm_max": nrm,
            "state_bytes": B * H * D * 2 * D * 4, "workspace_bytes": ws.numel(),
            "tflops_algorithmic": flops / (ms * 1e-3) / 1e12,
            "kernels": {n: {"avg_us": None if t is None else t * 1e3, "launches": c} for n, (t, c) in kern.items()},
            "pieces_16384": pieces}


# ----------------------------------------------------------------- CPU legs
def cpu_cores():
    n = len(os.sched_getaffinity(0))
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_inputs(nseq, H, L, seed):
    import numpy as np
    from oracle import oracle as O
    q, k, v = O.make_inputs((nseq, H, L, D), seed=seed, bf16=True)
    return q, k, v, np.random.default_rng(seed).uniform(0.99, 0.9999, H).astype(np.float32)


def cpu_prefill_legs(args):
    """Timed CPU baselines on bounded samples of the prefill workload; each
    leg grows its sample (whole sequences of L=8192 tokens x 12 heads) until
    about --cpu-budget seconds, capped at the workload's 8 sequences."""
    import numpy as np
    import torch
    from oracle import oracle as O
    from oracle import torch_cpu as T
    H, L, maxseq = 12, 8192, 8
    n = cpu_cores()
    q, k, v, lam = cpu_inputs(maxseq, H, L, args.seed)
    legs = []

    def grow(run_one, kind, cores, label):
        t0 = time.perf_counter()
        run_one(0)
        t1 = time.perf_counter() - t0
        done, total = 1, t1
        while done < maxseq and total + t1 < args.cpu_budget:
            t0 = time.perf_counter()
            run_one(done)
            total += time.perf_counter() - t0
            done += 1
        legs.append({"value": done * L / total, "unit": "tok/s", "cores": cores, "kind": kind,
                     "sample": f"{done} of 8 sequences x 12 heads x L=8192 of the prefill workload "
                               f"({done * L} tokens, {total:.2f} s)", "impl": label})

    if O.ref_available():
        def ref_one(i):
            e = O.RefEngine(H, D, 0.9995, 1.0)
            # the engine scales q by 1/sqrt(D) itself and walks tokens [L, H, D]
            e.prefill(np.ascontiguousarray((q[i] * 8).transpose(1, 0, 2)),
                      np.ascontiguousarray(k[i].transpose(1, 0, 2)),
                      np.ascontiguousarray(v[i].transpose(1, 0, 2)))
        grow(ref_one, "reference", 1, "reference C99 engine (c/prime_moment.c, additive mode, single "
             "decay 0.9995), built from the reference sources, 1 thread")

    def port_one(i):
        st = tuple(np.zeros(s, np.float32) for s in ((H, D), (H, D, D), (H, D, D), (H,), (H, D), (H, D)))
        y = np.empty((H, L, D), np.float32)
        O.baseline_prefill(np.ascontiguousarray(q[i]), np.ascontiguousarray(k[i]), np.ascontiguousarray(v[i]),
                           lam, 1.0, st, y, H, n)
    grow(port_one, "port", n, f"C restatement of c/prime_moment.c:276-312 with PyTorch semantics, "
         f"OpenMP over (sequence, head), {n} threads")

    torch.set_num_threads(n)

    def torch_one(i):
        t = lambda x: torch.from_numpy(np.ascontiguousarray(x[i:i + 1]))
        T.chunked_core(t(q), t(k), t(v), torch.from_numpy(lam), chunk=64, carry="dense")
    grow(torch_one, "port", n, f"PyTorch-CPU fp32 restatement of chunked_ssd.py:48-184 with the "
         f"reference's O(Nc^2) carry, torch threads {n}")
    return legs


def cpu_model_legs(args, model, ids, decode_states):
    """The fp32 PyTorch-CPU restatement of the same model (oracle/torch_cpu.py
    CausalLMCPU: the reference's layers and its chunked core with the O(Nc^2)
    carry) on the same weights, all host cores.  Prefill: whole sequences of
    the B=32 x 2048 workload, grown until about --cpu-budget seconds.  Decode:
    greedy steps at B=256 from the GPU's states after the 128-token prompt
    (a step's cost does not depend on the position), up to 8 steps or the
    budget."""
    import torch
    from oracle.torch_cpu import CausalLMCPU
    n = cpu_cores()
    torch.set_num_threads(n)
    cfg = model.config
    c = CausalLMCPU(model.state_dict(), cfg.num_layers, cfg.num_heads, cfg.head_dim, cfg.decay, eps=cfg.eps,
                    rms_eps=cfg.rms_norm_eps, qk_norm=cfg.use_qk_norm)
    ids_c = ids.cpu()
    impl = (f"fp32 PyTorch-CPU restatement of the reference model (model.py:47-200, attention through "
            f"chunked_ssd.py:48-184 with its O(Nc^2) carry, step attention.py:119-143), same weights, "
            f"torch threads {n}")
    done, total = 0, 0.0
    while done < ids_c.shape[0] and (done == 0 or total * (done + 1) / done < args.cpu_budget):
        t0 = time.perf_counter()
        c.prefill(ids_c[done:done + 1])
        total += time.perf_counter() - t0
        done += 1
    L = ids_c.shape[1]
    pre = {"value": done * L / total, "unit": "tok/s", "cores": n, "kind": "port",
           "sample": f"prefill of {done} of {ids_c.shape[0]} sequences x {L} tokens of the workload, one sequence "
                     f"per call ({done * L} tokens, {total:.2f} s)", "impl": impl}
    states = [tuple(t.detach().float().cpu() for t in st) for st in decode_states]
    Bd = states[0][0].shape[0]
    tok = torch.randint(0, cfg.vocab_size, (Bd,), generator=torch.Generator().manual_seed(args.seed))
    steps, total = 0, 0.0
    while steps < 8 and (steps == 0 or total * (steps + 1) / steps < args.cpu_budget):
        t0 = time.perf_counter()
        logits, states = c.step(tok, states)
        tok = logits.argmax(-1)
        total += time.perf_counter() - t0
        steps += 1
    dec = {"value": Bd * steps / total, "unit": "tok/s", "cores": n, "kind": "port",
           "sample": f"{steps} greedy decode steps at B={Bd} from the GPU's states after a 128-token prompt "
                     f"({total:.2f} s)", "impl": impl}
    return pre, dec


def cpu_decode_leg(args):
    """Reference C99 engine, one decode step per (sequence, layer) of the B=512
    x 12-layer x 12-head workload, 1 thread, on a bounded number of sequences."""
    import numpy as np
    from oracle import oracle as O
    if not O.ref_available():
        return None
    H, layers = 12, 12
    engines = [O.RefEngine(H, D, 0.9995, 1.0) for _ in range(layers)]
    rng = np.random.default_rng(args.seed)
    toks = rng.standard_normal((64, 3, H, D)).astype(np.float32)
    seqs, t_total, steps = 0, 0.0, 0
    t0 = time.perf_counter()
    while t_total < min(args.cpu_budget, 4.0):
        for e in engines:
            x = toks[steps % 64]
            e.step(x[0], x[1], x[2])
        steps += 1
        t_total = time.perf_counter() - t0
    # every (sequence, layer) pair costs the same: tokens/s over 512 sequences
    per_seq_step = t_total / steps
    return {"value": 1.0 / per_seq_step, "unit": "tok/s", "cores": 1, "kind": "reference",
            "sample": f"{steps} decode steps of one sequence through 12 layers x 12 heads "
                      f"({t_total:.2f} s); a 512-sequence step costs 512x this"}


# ----------------------------------------------------------------- main
def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py runs on ONE GPU only: the PRIME hot paths here are single-GPU kernels "
              "(sharding over (sequence, head) is a design note, not a built path). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch
    from prime_moment_attention import _lib as lib
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    lib.load()
    if args.copy_calibration:
        src = torch.ones(1 << 28, device=dev)   # 1 GiB of fp32
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # kernel-level legs first: they also bring the GPU clocks up before the headline
    hbm = bench_hbm(lib, torch, dev)
    ach = hbm["achievable_GBps"] * 1e9
    pf = bench_prefill(args, lib, torch, dev)
    main_s = pf["main_ms"] * 1e-3
    traffic = load_traffic().get("prefill_chunks")  # measured for this kernel at this workload
    kernels = {"prefill_config2": {
        "workload": "chunked prefill alone, BASELINE config 2: B=8 x H=12 x L=8192, D=64, chunk 64, bf16 q/k/v, "
                    "per-head lambda U[0.99,0.9999], zero initial state, bf16 y, fp32 final state",
        "tok_s": pf["tokens"] / (pf["ms"] * 1e-3), "ms_per_call": pf["ms"], "calls": args.kernel_steps,
        "workspace_bytes": pf["ws_bytes"], "finite": pf["finite"],
        "roofline": {"kernel": "prefill_bf16_kernel<false, false, true, true, false> (fused chunk loop, 16 waves)",
                     "bound": "hbm", "achieved": pf["bytes"] / main_s / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": pf["bytes"] / main_s / PEAK_HBM,
                     "traffic": None if traffic is None else traffic.get("bytes_per_launch"),
                     "bytes_per_launch": pf["bytes"], "avg_launch_us": pf["main_ms"] * 1e3,
                     "frac_of_measured": pf["bytes"] / main_s / ach},
        "whole_call_GBps": pf["bytes"] / (pf["ms"] * 1e-3) / 1e9,
        "whole_call_hbm_frac": pf["bytes"] / (pf["ms"] * 1e-3) / PEAK_HBM,
        "mfma_frac": pf["flops"] / (pf["ms"] * 1e-3) / PEAK_BF16,
        "kernels": pf["kernels"], "ms_per_call_with_events": pf["ms_events"]}}
    extra = {}
    if not args.no_decode:
        d512 = bench_decode(args, lib, torch, dev, B=512)
        d256 = bench_decode(args, lib, torch, dev, B=256)
        for d, key in ((d512, "decode_b512"), (d256, "decode_b256")):
            t = load_traffic().get(key)
            if t is not None:
                d["roofline"]["traffic"] = t.get("bytes_per_launch")
            d["roofline"]["frac_of_measured"] = d["roofline"]["achieved"] * 1e9 / ach
        extra["decode"] = {"B=512": d512, "B=256": d256}
    if not args.no_delta:
        extra["delta"] = bench_delta(args, lib, torch, dev)
    if not args.no_selective:
        extra["selective"] = bench_selective(args, lib, torch, dev)
    if not args.no_hybrid:
        extra["hybrid"] = bench_hybrid(args, lib, torch, dev)
    if not args.no_backward:
        extra["backward"] = bench_backward(args, lib, torch, dev)

    # the headline: PRIME-125M prefill (value) and greedy decode at B=256
    m = bench_model(args, lib, torch, dev)
    model, ids, dstates = m.pop("_model"), m.pop("_ids"), m.pop("_decode_states_B256")
    roof = m.pop("roofline")
    d256m = m["decode_B256"]
    rec = {
        "metric": "prefill tok/s + decode tok/s (B=256) PRIME-125M, 1 MI355X; % MFMA/HBM roofline",
        "value": m["prefill"]["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": m["prefill"]["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (uniform random token ids, random-init weights N(0, 0.02), seeded)",
        "config": {"workload": "PRIME-125M-shaped causal LM (12 layers, d_model 768, 12 heads x 64, GELU MLP 3072, "
                               "vocab 50304 tied, bf16 weights, fp32 states, LayerNorm QK-norm): value = prefill "
                               "tok/s of B=32 x 2048 (a step = one prefill: states and the last position's logits "
                               "and greedy token); decode_tok_s = greedy decode tok/s at B=256 (HIP-graph step)",
                   "prefill_batch": MODEL_B, "prefill_len": MODEL_L, "decode_batch": DECODE_B,
                   "decode_prompt": DECODE_PROMPT, "decode_steps": args.decode_steps, "seed": args.seed},
        "decode_tok_s": d256m["tok_s"],
        "decode_ms_per_step": d256m["ms_per_step"],
        "roofline": roof,
        "decode_roofline": d256m["roofline"],
        "model": m,
        "kernels": kernels,
        **extra,
        "hbm_measured": hbm,
        "gpu": f"{torch.cuda.get_device_name(dev)} ({torch.cuda.get_device_properties(dev).gcnArchName}, "
               f"{torch.cuda.get_device_properties(dev).multi_processor_count} CUs)",
        "gpu_clock": m.pop("gpu_clock"),
    }
    if not args.no_selective:
        rec["model_selective"] = bench_model_selective(args, torch, dev)
    if not args.no_cpu:
        try:
            pre, dec = cpu_model_legs(args, model, ids, dstates)
            rec["cpu_baseline"] = pre
            rec["decode_cpu_baseline"] = dec
            rec["cpu_model"] = cpu_model()
        except Exception as exc:  # the GPU figures stand without the CPU legs
            rec["cpu_baseline"] = None
            rec["cpu_baseline_error"] = f"{type(exc).__name__}: {exc}"
        try:
            legs = cpu_prefill_legs(args)
            ref = [x for x in legs if x["kind"] == "reference"]
            kernels["prefill_config2"]["cpu_baseline"] = ref[0] if ref else legs[0]
            kernels["prefill_config2"]["cpu_baselines"] = legs
            if not args.no_decode:
                rec["decode"]["cpu_baseline"] = cpu_decode_leg(args)
        except Exception as exc:
            kernels["prefill_config2"]["cpu_baseline_error"] = f"{type(exc).__name__}: {exc}"
    detail = args.detail
    if detail is None and os.path.isdir(os.path.join(ROOT, "gpurun_out")):
        detail = os.path.join(ROOT, "gpurun_out", "bench_full.json")
    if detail:
        with open(detail, "w") as f:
            json.dump(rec, f, indent=1, default=str)
    print(json.dumps(compact(rec), separators=(",", ":")), flush=True)
    return 0


def _r(x, nd=4):
    """Round a float to nd significant digits for the printed record."""
    if isinstance(x, float):
        return float(f"{x:.{nd}g}")
    if isinstance(x, dict):
        return {k: _r(v, nd) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return [_r(v, nd) for v in x]
    return x


def _roof(r, keys=("bound", "achieved", "peak", "unit", "frac", "traffic")):
    return None if r is None else {k: r.get(k) for k in keys if k in r}


def compact(rec):
    """The printed record: the driver keeps the tail of stdout, so the line
    stays under about 6 KB with every headline figure (prefill and decode
    rooflines, the kernel-level legs, the CPU baselines); the full record goes
    to --detail."""
    out = {k: rec[k] for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                               "higher_is_better", "scaling", "vs_baseline", "dtype", "data")}
    cfg = dict(rec["config"])
    cfg["workload"] = ("PRIME-125M-shaped LM (12L, d768, 12x64 heads, GELU MLP 3072, vocab 50304 tied, bf16 "
                       "weights, fp32 states, LN QK-norm); value = prefill tok/s of B=32x2048 (a step = one "
                       "prefill with states, last-position logits and greedy token); decode_tok_s = greedy "
                       "decode at B=256 (HIP-graph step)")
    out["config"] = cfg
    out["roofline"] = _roof(rec["roofline"], ("bound", "achieved", "peak", "unit", "frac", "traffic",
                                              "flop_per_step", "avg_step_ms"))
    cb = rec.get("cpu_baseline")
    out["cpu_baseline"] = None if cb is None else {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    if "cpu_baseline_error" in rec:
        out["cpu_baseline_error"] = rec["cpu_baseline_error"][:200]
    out["decode_tok_s"] = rec["decode_tok_s"]
    out["decode_ms_per_step"] = rec["decode_ms_per_step"]
    out["decode_roofline"] = _roof(rec["decode_roofline"], ("bound", "achieved", "peak", "unit", "frac",
                                                           "bytes_per_step"))
    m = rec["model"]
    out["decode_B32"] = {"tok_s": m["decode_B32"]["tok_s"], "ms_per_step": m["decode_B32"]["ms_per_step"]}
    dcb = rec.get("decode_cpu_baseline")
    if dcb:
        out["decode_cpu_baseline"] = {k: dcb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    ar = m["prefill"]["attention_roofline"]
    out["prefill_attention"] = {"us_per_layer": m["prefill"]["attention_us_per_layer"],
                                "fused_kernel_us": ar["avg_launch_us"], "hbm_frac": ar["frac"]}
    k2 = rec["kernels"]["prefill_config2"]
    c2 = {"tok_s": k2["tok_s"], "ms_per_call": k2["ms_per_call"], "roofline": _roof(k2["roofline"]),
          "kernel_us": k2["roofline"]["avg_launch_us"], "frac_of_measured": k2["roofline"]["frac_of_measured"],
          "whole_call_hbm_frac": k2["whole_call_hbm_frac"], "mfma_frac": k2["mfma_frac"]}
    c2cb = k2.get("cpu_baseline")
    if c2cb:
        c2["cpu_baseline"] = {k: c2cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    out["config2_prefill"] = c2
    if "decode" in rec:
        d = rec["decode"]
        out["config3_decode"] = {
            b: {"tok_s": d[b]["tok_s"], "ms_per_step": d[b]["ms_per_step"], "roofline": _roof(d[b]["roofline"]),
                "kernel_us": d[b]["roofline"]["avg_launch_us"],
                "frac_of_measured": d[b]["roofline"].get("frac_of_measured")} for b in ("B=512", "B=256")}
        if d.get("cpu_baseline"):
            out["config3_decode"]["cpu_baseline"] = {k: d["cpu_baseline"][k]
                                                     for k in ("value", "unit", "cores", "kind", "sample")}
    if "delta" in rec:
        dl = rec["delta"]
        pt = [p["tok_s"] for p in dl["pieces_16384"]]
        mem = [p["mem_allocated_MB"] for p in dl["pieces_16384"]]
        out["config5_delta"] = {"tok_s": dl["tok_s"], "ms": dl["ms"], "piece_tok_s_min": min(pt),
                                "piece_tok_s_max": max(pt), "mem_MB_min": min(mem), "mem_MB_max": max(mem),
                                "state_norm_max": dl["state_norm_max"],
                                "kernel_us": {k: v["avg_us"] for k, v in dl["kernels"].items()}}
    if "selective" in rec:
        se = rec["selective"]
        out["selective"] = {"prefill_tok_s": se["prefill"]["tok_s"], "prefill_ms": se["prefill"]["ms"],
                            "prefill_f32_ms": se["prefill_f32"]["ms"],
                            "prefill_hbm_frac": se["prefill"]["roofline"]["frac"],
                            "decode_B256_tok_s": se["decode_B256"]["tok_s"],
                            "decode_hbm_frac": se["decode_B256"]["roofline"]["frac"]}
    if "hybrid" in rec:
        out["hybrid"] = {k: {"tok_s": v["tok_s"], "hbm_frac": v["roofline"]["frac"]} for k, v in rec["hybrid"].items()}
    if "backward" in rec:
        out["backward"] = {k: {"ms": v["ms"], "tok_s": v["tok_s"], "hbm_frac": v["roofline"]["hbm_frac"],
                               "mfma_frac": v["roofline"]["mfma_frac"]} for k, v in rec["backward"].items()}
    if "model_selective" in rec:
        ms = rec["model_selective"]
        out["model_selective"] = {"prefill_tok_s": ms["prefill"]["tok_s"], "decode_B256_tok_s": ms["decode_B256"]["tok_s"]}
    h = rec["hbm_measured"]
    out["hbm_measured"] = {k: h[k] for k in ("copy_GBps", "read_GBps", "achievable_GBps")}
    out["gpu"] = rec["gpu"]
    gc = rec.get("gpu_clock") or {}
    out["gpu_clock"] = {k: (v.get("gfx_mhz") or v.get("cards") or v.get("error")) if isinstance(v, dict) else v
                        for k, v in gc.items()}
    if "cpu_model" in rec:
        out["cpu_model"] = rec["cpu_model"]
    exact = {k: out[k] for k in ("value", "ms_per_step", "decode_tok_s", "decode_ms_per_step")}
    out = _r(out)
    out.update(exact)
    return out


if __name__ == "__main__":
    sys.exit(main())
