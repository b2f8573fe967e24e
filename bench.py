"""Benchmark of the gfx950 full-attention path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Headline line (one JSON object on stdout): decode attention GB/s at 8K KV, on the workload
"decode_8k_batch32": 32 sequences x (16 query heads, 4 kv heads, head_dim 256), 8192 fp16 KV rows each
(the last one appended by the step), one query token per sequence, sigmoid gate, fp32 q/gate/out.
A step is one bn_attn_decode_ragged call over the batch; its inputs are resident in HBM before timing.
Algorithmic bytes per sequence: K/V read 8192*4*256*2*2 + q, gate, out fp32 (3*16*256*4) + new K/V fp32
(2*4*256*4) + fp16 append (2*4*256*2) = 33,615,872 B; 32 sequences = 1,075,707,904 B per step (> the
256 MB last-level cache, so the rate is an HBM rate).
The same line carries the prefill figure (TFLOP/s against the dense fp16 MFMA peak) for "prefill_4k":
4096 causal rows from an empty cache, 16 query heads, 4 kv heads; FLOPs = 4*H*256*sum_t(t+1).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2516.6
D = 256


def load_package():
    import importlib.util
    pkg_dir = os.path.join(ROOT, "glimpse-language_amd")
    if "glimpse_language_amd" in sys.modules:
        return sys.modules["glimpse_language_amd"]
    spec = importlib.util.spec_from_file_location("glimpse_language_amd", os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["glimpse_language_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def decode_bytes(nseq, H, KV, L):
    per = L * KV * D * 2 * 2 + 3 * H * D * 4 + 2 * KV * D * 4 + 2 * KV * D * 2
    return nseq * per


def prefill_flops(H, T, off):
    return 4 * H * D * sum(off + t + 1 for t in range(T))


def rms(torch, x):
    return x * torch.rsqrt((x.double() ** 2).mean(-1, keepdim=True) + 1e-6).float()


def time_steps(torch, fn, steps, warmup):
    """Runs warmup untimed steps, then `steps` timed ones bracketed by synchronisations; per-step HIP events
    on the launch stream (torch's current stream) give the average step (kernel) duration."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(steps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    total_ms = ev[0].elapsed_time(ev[steps])
    return total_ms / steps, per, wall


def bench_decode(torch, ba, ctx, steps, warmup, nseq=32, H=16, KV=4, L=8192):
    g = torch.Generator(device="cuda")
    g.manual_seed(0xB0A5A104)
    dev = "cuda"
    kc = rms(torch, torch.randn(nseq * L, KV, D, device=dev, generator=g)).half().view(torch.int16)
    vc = torch.randn(nseq * L, KV, D, device=dev, generator=g).half().view(torch.int16)
    q = rms(torch, torch.randn(nseq, H, D, device=dev, generator=g))
    k_new = rms(torch, torch.randn(nseq, KV, D, device=dev, generator=g))
    v_new = torch.randn(nseq, KV, D, device=dev, generator=g)
    gate = torch.randn(nseq, H, D, device=dev, generator=g)
    kv_off = torch.arange(nseq, device=dev, dtype=torch.int64) * L
    kv_len = torch.full((nseq,), L, device=dev, dtype=torch.int32)
    out = torch.empty(nseq, H, D, device=dev)
    ws = ba.Workspace(ctx, dev)

    def step():
        ba.decode_ragged(ctx, ws, q, kc, vc, kv_off, kv_len, L, out=out, k_new=k_new, v_new=v_new, gate=gate)

    ms, per, wall = time_steps(torch, step, steps, warmup)
    nbytes = decode_bytes(nseq, H, KV, L)
    kernel_ms = sum(per) / len(per)
    return dict(ms=ms, kernel_ms=kernel_ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9,
                kernel_gbs=nbytes / (kernel_ms * 1e-3) / 1e9, wall=wall)


def bench_prefill(torch, ba, ctx, steps, warmup, H=16, KV=4, T=4096, off=0):
    g = torch.Generator(device="cuda")
    g.manual_seed(0xB0A5A103)
    dev = "cuda"
    cap = off + T
    kc = torch.zeros(cap, KV, D, device=dev, dtype=torch.int16)
    vc = torch.zeros(cap, KV, D, device=dev, dtype=torch.int16)
    q = rms(torch, torch.randn(T, H, D, device=dev, generator=g)).half().float()
    k_new = rms(torch, torch.randn(T, KV, D, device=dev, generator=g)).half().float()
    v_new = torch.randn(T, KV, D, device=dev, generator=g).half().float()
    gate = torch.randn(T, H, D, device=dev, generator=g)
    out = torch.empty(T, H, D, device=dev)
    ws = ba.Workspace(ctx, dev)

    def step():
        ba.attention(ctx, ws, q, kc, vc, off, out=out, k_new=k_new, v_new=v_new, gate=gate, kind=ba.KIND_PREFILL)

    ms, per, wall = time_steps(torch, step, steps, warmup)
    flops = prefill_flops(H, T, off)
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12, wall=wall)


def cpu_baseline(budget_s=10.0, H=16, KV=4, L=8192, nseq=2):
    """The oracle (scalar C restatement of the reference shaders, OpenMP over its work units) on a bounded
    sample of the decode workload, on this host's cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle
    threads = min(16, os.cpu_count() or 1)
    rows = nseq * L
    kc = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(0xB0A5A104, 2, (rows, KV, D))))
    vc = oracle.f32_to_f16(oracle.normal(0xB0A5A104, 3, (rows, KV, D)))
    q = oracle.rms_rows(oracle.normal(0xB0A5A104, 1, (nseq, H, D)))
    z = oracle.normal(0xB0A5A104, 6, (nseq, H, D))
    offs = np.arange(nseq, dtype=np.int64) * L
    lens = np.full(nseq, L, dtype=np.int32)
    reps, t = 0, 0.0
    while t < budget_s or reps == 0:
        t0 = time.perf_counter()
        oracle.decode_ragged(q, kc, vc, offs, lens, z, nthreads=threads)
        t += time.perf_counter() - t0
        reps += 1
    nbytes = decode_bytes(nseq, H, KV, L) * reps
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{nseq} of the 32 sequences x {reps} reps ({t:.1f} s): oracle in shader order "
                      f"(oracle/bn_oracle.c, -O2, no fast-math), OpenMP {threads} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the attention path has no cross-GPU exchange); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    ba = load_package().bonsai_attn
    ctx = ba.Context(0)
    print(f"bench: decode_8k_batch32 steps={args.steps} warmup={args.warmup}", file=sys.stderr, flush=True)
    dec = bench_decode(torch, ba, ctx, args.steps, args.warmup)
    print(f"bench: decode {dec['gbs']:.1f} GB/s ({dec['ms']*1e3:.1f} us/step)", file=sys.stderr, flush=True)
    pre = None
    if not args.no_prefill:
        print("bench: prefill_4k", file=sys.stderr, flush=True)
        pre = bench_prefill(torch, ba, ctx, max(2, args.steps // 4), max(1, args.warmup // 2))
        print(f"bench: prefill {pre['tflops']:.1f} TFLOP/s ({pre['ms']:.3f} ms/step)", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        print("bench: cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline()
    line = {
        "metric": "attn decode GB/s (%HBM peak) @8K KV; prefill TFLOP/s (%MFMA peak)",
        "value": round(dec["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV, f32 accumulate",
        "data": "synthetic (seeded: RMS-normalised N(0,1) q/k rows, N(0,1) v and gate logits)",
        "config": {"workload": "decode_8k_batch32", "sequences": 32, "q_heads": 16, "kv_heads": 4,
                   "head_dim": 256, "kv_rows_per_sequence": 8192, "kv_dtype": "fp16", "append": True,
                   "gate": True, "hbm_peak_frac": round(dec["gbs"] / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(dec["kernel_gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec["kernel_gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "bn::decode_kernel", "algorithmic_bytes": dec["bytes"]},
        "cpu_baseline": cpu,
    }
    if pre:
        line["prefill"] = {"workload": "prefill_4k", "value": round(pre["tflops"], 3), "unit": "TFLOP/s",
                           "ms_per_step": round(pre["ms"], 5), "flops": pre["flops"], "peak": MFMA_F16_PEAK_TFLOPS,
                           "frac": round(pre["tflops"] / MFMA_F16_PEAK_TFLOPS, 5)}
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
