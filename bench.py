"""Benchmark of the gfx950 full-attention path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--only NAMES] [--copy-calib MB]

Headline line (one JSON object on stdout): decode attention GB/s at 8K KV, on the workload
"decode_8k_batch32": 32 sequences x (16 query heads, 4 kv heads, head_dim 256), 8192 fp16 KV rows each
(the last one appended by the step), one query token per sequence, sigmoid gate, fp32 q/gate/out.
A step is one bn_attn_decode_ragged call over the batch; its inputs are resident in HBM before timing.
Algorithmic bytes per sequence: K/V read 8192*4*256*2*2 + q, gate, out fp32 (3*16*256*4) + new K/V fp32
(2*4*256*4) + fp16 append (2*4*256*2) = 33,615,872 B; 32 sequences = 1,075,707,904 B per step (> the
256 MB last-level cache, so the rate is an HBM rate).
The same line carries the prefill figure (TFLOP/s against the dense fp16 MFMA peak) for "prefill_4k":
4096 causal rows from an empty cache, 16 query heads, 4 kv heads, fp16 q (fp32 gate and output, new K/V rows
fp32 rounded to fp16 by the call); FLOPs = 4*H*256*sum_t(t+1), and the
other workloads (ragged decode, verify, short decode, prefill over a cached prefix) under "workloads".

--copy-calib MB runs a plain device copy of MB MiB (three times) before the workloads: its kernel gives the
bytes-per-count scale of the FETCH_SIZE / WRITE_SIZE counters when the run is profiled.
"""
import argparse
import json
import os
import shutil
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


def decode_bytes(H, KV, lens):
    """Algorithmic bytes of single-token decodes: fp16 K/V rows read, q/gate/out fp32, new K/V fp32 in, fp16 out."""
    per_seq = 3 * H * D * 4 + 2 * KV * D * 4 + 2 * KV * D * 2
    return sum(L * KV * D * 2 * 2 for L in lens) + len(lens) * per_seq


def attn_bytes(H, KV, T, off, q_bytes=4):
    """Algorithmic bytes of a T-row call: cache rows [0, off) read once, q (q_bytes/elem), gate and out fp32,
    new K/V fp32 in and fp16 out (the new rows are then read from the cache in fp16)."""
    return (off * KV * D * 2 * 2 + T * H * D * (q_bytes + 4 + 4) + T * KV * D * 2 * (4 + 2) + T * KV * D * 2 * 2)


def attn_flops(H, T, off):
    return 4 * H * D * sum(off + t + 1 for t in range(T))


def rms(torch, x):
    return x * torch.rsqrt((x.double() ** 2).mean(-1, keepdim=True) + 1e-6).float()


def time_steps(torch, fn, steps, warmup):
    """Runs `warmup` untimed steps, then `steps` timed ones bracketed by synchronisations. Two HIP events recorded
    on the launch stream (torch's current stream, where the library launches) around the timed steps give the
    average step duration; a step is one library call with its argument structs built beforehand (as a compiled
    caller holds them), so host-side Python does not pace the small calls."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps, wall


def _gen(torch, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


RAGGED_SEED = 0xB0A5A104


def ragged_lengths(nseq=32, lo=1024, hi=32768, seed=RAGGED_SEED):
    """KV lengths of the ragged batch: uniform integers in [lo, hi] from Python's seeded generator
    (32 sequences: sum 507,255)."""
    import random
    rng = random.Random(seed)
    return [rng.randint(lo, hi) for _ in range(nseq)]


def decode_batch_inputs(torch, lens, H=16, KV=4, seed=0xB0A5A104):
    """Device inputs of a batch of single-token decodes (one sequence per entry of `lens`, rows contiguous):
    RMS-normalised N(0,1) K rows and q, N(0,1) V rows, new K/V rows and gate logits, drawn on the GPU."""
    g = _gen(torch, seed)
    nseq, rows = len(lens), sum(lens)
    kc = rms(torch, torch.randn(rows, KV, D, device="cuda", generator=g)).half().view(torch.int16)
    vc = torch.randn(rows, KV, D, device="cuda", generator=g).half().view(torch.int16)
    q = rms(torch, torch.randn(nseq, H, D, device="cuda", generator=g))
    k_new = rms(torch, torch.randn(nseq, KV, D, device="cuda", generator=g))
    v_new = torch.randn(nseq, KV, D, device="cuda", generator=g)
    gate = torch.randn(nseq, H, D, device="cuda", generator=g)
    offs = [0]
    for L in lens[:-1]:
        offs.append(offs[-1] + L)
    kv_off = torch.tensor(offs, device="cuda", dtype=torch.int64)
    kv_len = torch.tensor(lens, device="cuda", dtype=torch.int32)
    return dict(kc=kc, vc=vc, q=q, k_new=k_new, v_new=v_new, gate=gate, kv_off=kv_off, kv_len=kv_len)


def attn_inputs(torch, H, KV, T, off, seed, q_f16=False):
    """Device inputs of one T-row attention call over `off` cached rows (cap = off + T), drawn on the GPU as
    decode_batch_inputs; q as fp16 when q_f16 (passed with BN_Q_F16)."""
    g = _gen(torch, seed)
    cap = off + T
    kc = rms(torch, torch.randn(cap, KV, D, device="cuda", generator=g)).half().view(torch.int16)
    vc = torch.randn(cap, KV, D, device="cuda", generator=g).half().view(torch.int16)
    q = rms(torch, torch.randn(T, H, D, device="cuda", generator=g))
    if q_f16:
        q = q.half()
    k_new = rms(torch, torch.randn(T, KV, D, device="cuda", generator=g))
    v_new = torch.randn(T, KV, D, device="cuda", generator=g)
    gate = torch.randn(T, H, D, device="cuda", generator=g)
    return dict(kc=kc, vc=vc, q=q, k_new=k_new, v_new=v_new, gate=gate)


class Workloads:
    def __init__(self, torch, ba, ctx):
        self.torch, self.ba, self.ctx = torch, ba, ctx
        self.ws = ba.Workspace(ctx, "cuda")

    def _gen(self, seed):
        g = self.torch.Generator(device="cuda")
        g.manual_seed(seed)
        return g

    def signs(self, H, seed=0xB0A5A1FF):
        g = self._gen(seed)
        return self.torch.randint(0, 2, (H * D,), device="cuda", generator=g).float() * 2 - 1

    def decode_batch(self, steps, warmup, nseq=32, H=16, KV=4, lens=None, seed=0xB0A5A104, rotate=False):
        torch, ba, ctx = self.torch, self.ba, self.ctx
        if lens is None:
            lens = [8192] * nseq
        nseq = len(lens)
        x = decode_batch_inputs(torch, lens, H, KV, seed)
        kc, vc, q, k_new, v_new, gate = x["kc"], x["vc"], x["q"], x["k_new"], x["v_new"], x["gate"]
        kv_off, kv_len = x["kv_off"], x["kv_len"]
        out = torch.empty(nseq, H, D, device="cuda")
        max_len = max(lens)
        signs = self.signs(H) if rotate else None

        a, _ = ba.decode_ragged_args(ctx, self.ws, q, kc, vc, kv_off, kv_len, max_len, out=out, k_new=k_new,
                                     v_new=v_new, gate=gate, signs=signs)
        step = ba.bind(ctx, "bn_attn_decode_ragged", a)

        ms, wall = time_steps(torch, step, steps, warmup)
        nbytes = decode_bytes(H, KV, lens)
        del kc, vc
        return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9, wall=wall)

    def attn(self, steps, warmup, H, KV, T, off, kind, seed, q_f16=False, rotate=False):
        torch, ba, ctx = self.torch, self.ba, self.ctx
        x = attn_inputs(torch, H, KV, T, off, seed, q_f16)
        kc, vc, q, k_new, v_new, gate = x["kc"], x["vc"], x["q"], x["k_new"], x["v_new"], x["gate"]
        out = torch.empty(T, H, D, device="cuda")
        signs = self.signs(H) if rotate else None

        a, _ = ba.attention_args(ctx, self.ws, q, kc, vc, off, out=out, k_new=k_new, v_new=v_new, gate=gate,
                                 signs=signs)
        step = ba.bind(ctx, ba._KIND_FN[kind], a)

        ms, wall = time_steps(torch, step, steps, warmup)
        flops = attn_flops(H, T, off)
        nbytes = attn_bytes(H, KV, T, off, q_bytes=2 if q_f16 else 4)
        return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12, bytes=nbytes,
                    gbs=nbytes / (ms * 1e-3) / 1e9, wall=wall)


    def prep(self, steps, warmup, H, KV, T, off, seed=0xB0A5A106):
        """bn_attn_prep over T rows: q_proj output [T][H][512] (q half read), k/v_proj rows, norm weights,
        positions; q out fp32, fp16 K/V rows written at [off, off + T)."""
        torch, ba, ctx = self.torch, self.ba, self.ctx
        g = self._gen(seed)
        qp = torch.randn(T, H, 512, device="cuda", generator=g)
        kp = torch.randn(T, KV, D, device="cuda", generator=g)
        vp = torch.randn(T, KV, D, device="cuda", generator=g)
        qn = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
        kn = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
        p = torch.arange(off, off + T, device="cuda", dtype=torch.int32)
        pos = torch.stack([p, p, p]).contiguous()
        inv = 1.0 / (1e7 ** (torch.arange(32, device="cuda", dtype=torch.float32) * 2 / 64))
        kc = torch.empty(off + T, KV, D, device="cuda", dtype=torch.int16)
        vc = torch.empty_like(kc)
        q = torch.empty(T, H, D, device="cuda")

        step = ba.bind(ctx, "bn_attn_prep", ba.prep_args(qp, kp, vp, qn, kn, pos, inv, q, kc, vc, off))

        ms, wall = time_steps(torch, step, steps, warmup)
        nbytes = T * H * D * 4 * 2 + T * KV * D * 4 * 2 + T * KV * D * 2 * 2 + 3 * T * 4
        return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9, wall=wall)

    def rotate(self, steps, warmup, H, T, seed=0xB0A5A107):
        """bn_gate_rotate over T rows: attn [T][H*256] and the gate half of the q_proj output read, xr written."""
        torch, ba, ctx = self.torch, self.ba, self.ctx
        g = self._gen(seed)
        attn = torch.randn(T, H * D, device="cuda", generator=g)
        qp = torch.randn(T, H, 512, device="cuda", generator=g)
        signs = self.signs(H)
        xr = torch.empty(T, H * D, device="cuda")

        step = ba.bind(ctx, "bn_gate_rotate", ba.rotate_args(attn, signs, xr, qp[:, :, D:]))

        ms, wall = time_steps(torch, step, steps, warmup)
        nbytes = 3 * T * H * D * 4 + H * D * 4
        return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9, wall=wall)


    def layer(self, steps, warmup, H, KV, T, off, seed=0xB0A5A108):
        """bn_attn_layer: attn_prep + attention + gate + rotation in one call, from raw q_proj / k_proj / v_proj
        rows (q_proj's output [T][H][512], its second half the gate logits)."""
        torch, ba, ctx = self.torch, self.ba, self.ctx
        g = self._gen(seed)
        cap = off + T
        kc = rms(torch, torch.randn(cap, KV, D, device="cuda", generator=g)).half().view(torch.int16)
        vc = torch.randn(cap, KV, D, device="cuda", generator=g).half().view(torch.int16)
        qp = torch.randn(T, H, 512, device="cuda", generator=g)
        kp = torch.randn(T, KV, D, device="cuda", generator=g)
        vp = torch.randn(T, KV, D, device="cuda", generator=g)
        qn = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
        kn = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
        p = torch.arange(off, off + T, device="cuda", dtype=torch.int32)
        pos = torch.stack([p, p, p]).contiguous()
        inv = 1.0 / (1e7 ** (torch.arange(32, device="cuda", dtype=torch.float32) * 2 / 64))
        signs = self.signs(H)
        out = torch.empty(T, H, D, device="cuda")
        # a prefill's q goes through an fp16 scratch (BN_Q_F16), the form prefill_kernel reads fastest
        q = torch.empty(T, H, D, device="cuda", dtype=torch.float16) if T > ba.VERIFY_MAX else None

        pa, la, _ = ba.attention_layer_args(ctx, self.ws, qp, kp, vp, qn, kn, pos, inv, kc, vc, off, gate=qp[:, :, D:],
                                            signs=signs, out=out, q=q)
        step = ba.bind(ctx, "bn_attn_layer", pa, la)

        ms, wall = time_steps(torch, step, steps, warmup)
        flops = attn_flops(H, T, off)
        # cache rows read once (fp16), q half and gate half of q_proj, out, k/v rows in (fp32) and fp16 rows out
        nbytes = (off * KV * D * 2 * 2 + T * H * D * (4 + 4 + 4) + T * KV * D * 2 * (4 + 2) + T * KV * D * 2 * 2
                  + H * D * 4)
        return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12, bytes=nbytes,
                    gbs=nbytes / (ms * 1e-3) / 1e9, wall=wall)


    def kv_copy(self, steps, warmup, n_layers, KV, length, cap, seed=0xB0A5A109):
        """bn_kv_copy: the used rows of n_layers fp16 caches into a prefix-sized snapshot (encode_copy_state)."""
        torch, ba, ctx = self.torch, self.ba, self.ctx
        g = self._gen(seed)
        kc = torch.randn(n_layers, cap, KV, D, device="cuda", generator=g).half().view(torch.int16)
        vc = torch.randn(n_layers, cap, KV, D, device="cuda", generator=g).half().view(torch.int16)
        sk = torch.empty(n_layers, length, KV, D, device="cuda", dtype=torch.int16)
        sv = torch.empty_like(sk)
        src, dst = ba.kv_state(kc, vc, length), ba.kv_state(sk, sv, 0)

        step = ba.bind(ctx, "bn_kv_copy", src, dst)

        ms, wall = time_steps(torch, step, steps, warmup)
        nbytes = 2 * 2 * n_layers * length * KV * D * 2  # K and V, read and written
        return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9, wall=wall)


    def ternary(self, steps, warmup, T, K, os, add=False, seed=0xB0A5A10A):
        """bn_ternary_matmul: y_i (+)= x W_i^T for the matrices sharing x (random 2-bit codes, fp16 scales)."""
        torch, ba, ctx = self.torch, self.ba, self.ctx
        g = self._gen(seed)
        x = torch.randn(T, K, device="cuda", generator=g)
        mats = []
        for o in os:
            w = torch.randint(-2 ** 31, 2 ** 31 - 1, (o, K // 16), device="cuda", dtype=torch.int32, generator=g)
            sc = (0.02 * torch.rand(o, K // 128, device="cuda", generator=g) + 0.005).half().view(torch.int16)
            mats.append((w, sc, torch.zeros(T, o, device="cuda")))

        work = ba.ternary_workspace(x)  # T > 32: x split once per call
        step = ba.bind(ctx, "bn_ternary_matmul", ba.ternary_args(x, mats, add, work=work))

        ms, wall = time_steps(torch, step, steps, warmup)
        O = sum(os)
        # codes and scales read once, x read, y written (and read with add)
        nbytes = O * K // 4 + O * (K // 128) * 2 + T * K * 4 + T * O * 4 * (2 if add else 1)
        flops = 2 * T * K * O
        return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9, flops=flops,
                    tflops=flops / (ms * 1e-3) / 1e12, wall=wall)


    def block(self, steps, warmup, T, off, hid=2560, H=16, KV=4, seed=0xB0A5A10B):
        """One whole attention layer of the 4B model: norm_rotate, the q/k/v projections (one call), bn_attn_layer
        (prep, attention over the fp16 cache, gate, rotation) and o_proj added into the hidden rows: four library
        calls, their argument structs built once."""
        import ctypes
        torch, ba, ctx = self.torch, self.ba, self.ctx
        g = self._gen(seed)
        cap = off + T
        h = torch.randn(T, hid, device="cuda", generator=g)
        in_w = 1 + 0.1 * torch.randn(hid, device="cuda", generator=g)
        s_in, s_o = self.signs(hid // D, seed + 1), self.signs(H, seed + 2)

        def lin(o, k):
            w = torch.randint(-2 ** 31, 2 ** 31 - 1, (o, k // 16), device="cuda", dtype=torch.int32, generator=g)
            return w, (0.02 * torch.rand(o, k // 128, device="cuda", generator=g) + 0.005).half().view(torch.int16)

        wq, wk, wv, wo = lin(2 * H * D, hid), lin(KV * D, hid), lin(KV * D, hid), lin(hid, H * D)
        kc = rms(torch, torch.randn(cap, KV, D, device="cuda", generator=g)).half().view(torch.int16)
        vc = torch.randn(cap, KV, D, device="cuda", generator=g).half().view(torch.int16)
        qn = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
        kn = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
        p = torch.arange(off, off + T, device="cuda", dtype=torch.int32)
        pos = torch.stack([p, p, p]).contiguous()
        inv = 1.0 / (1e7 ** (torch.arange(32, device="cuda", dtype=torch.float32) * 2 / 64))
        xr = torch.empty(T, hid, device="cuda")
        qp = torch.empty(T, H, 512, device="cuda")
        kp = torch.empty(T, KV, D, device="cuda")
        vp = torch.empty(T, KV, D, device="cuda")
        q16 = torch.empty(T, H, D, device="cuda", dtype=torch.float16) if T > ba.VERIFY_MAX else None
        na = ba.norm_args(h, in_w, s_in, xr)
        qa = ba.ternary_args(xr, [(*wq, qp.view(T, -1)), (*wk, kp.view(T, -1)), (*wv, vp.view(T, -1))],
                             work=ba.ternary_workspace(xr))
        pa, la, xo = ba.attention_layer_args(ctx, self.ws, qp, kp, vp, qn, kn, pos, inv, kc, vc, off,
                                             gate=qp[:, :, D:], signs=s_o, q=q16)
        oa = ba.ternary_args(xo.view(T, H * D), [(*wo, h)], add=True, work=ba.ternary_workspace(xo.view(T, H * D)))
        st, L, by = ctx._stream(None), ctx.lib, ctypes.byref

        def step():
            ctx._check(L.bn_norm_rotate(ctx.h, st, by(na)), "bn_norm_rotate")
            ctx._check(L.bn_ternary_matmul(ctx.h, st, by(qa)), "bn_ternary_matmul")
            ctx._check(L.bn_attn_layer(ctx.h, st, by(pa), by(la)), "bn_attn_layer")
            ctx._check(L.bn_ternary_matmul(ctx.h, st, by(oa)), "bn_ternary_matmul")

        ms, wall = time_steps(torch, step, steps, warmup)
        O = 2 * H * D + 2 * KV * D
        w_bytes = (O * hid + hid * H * D) // 4 + (O * hid + hid * H * D) // 128 * 2
        # weights (codes, scales) and the cache rows read once; hidden rows read and written
        nbytes = w_bytes + off * KV * D * 2 * 2 + T * hid * 4 * 3
        flops = 2 * T * (O * hid + hid * H * D) + attn_flops(H, T, off)
        return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9, flops=flops,
                    tflops=flops / (ms * 1e-3) / 1e12, wall=wall)


def measured_traffic(name):
    """HBM bytes per step from a committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary under profiles/ (its
    `traffic_bytes_per_step:` line), or (None, None) when the summary is absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_step:"):
                return int(line.split(":")[1]), "profiles/" + name
    except OSError:
        pass
    return None, None


def copy_calibration(torch, mib):
    """A plain device-to-device copy of `mib` MiB, three times (reads and writes mib MiB per launch)."""
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def host_info():
    """The host the CPU baseline ran on: CPUs this process may use, the CPU model, and whether the reference's own
    Vulkan path could run here (a SPIR-V compiler for its shaders and a Vulkan driver manifest)."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    icds = []
    for d in ("/usr/share/vulkan/icd.d", "/etc/vulkan/icd.d", "/usr/local/share/vulkan/icd.d"):
        if os.path.isdir(d):
            icds += sorted(os.listdir(d))
    tools = {t: shutil.which(t) is not None for t in ("glslc", "glslangValidator", "vulkaninfo")}
    return {"nproc": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count(), "cpu_model": model,
            "vulkan_icds": icds, "shader_tools": tools,
            "reference_vulkan_path": "runnable" if icds and (tools["glslc"] or tools["glslangValidator"])
            else "not runnable here (no Vulkan driver manifest or no SPIR-V compiler)"}


def cpu_baseline(budget_s=8.0, H=16, KV=4, L=8192, nseq=4):
    """The oracle (scalar C restatement of the reference shaders, OpenMP over its work units) on a bounded
    sample of the decode workload: on this process's CPUs (at most 16, the box's share for one GPU) and on one
    core, each for about budget_s seconds."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle
    rows = nseq * L
    kc = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(0xB0A5A104, 2, (rows, KV, D))))
    vc = oracle.f32_to_f16(oracle.normal(0xB0A5A104, 3, (rows, KV, D)))
    q = oracle.rms_rows(oracle.normal(0xB0A5A104, 1, (nseq, H, D)))
    z = oracle.normal(0xB0A5A104, 6, (nseq, H, D))
    offs = np.arange(nseq, dtype=np.int64) * L
    lens = np.full(nseq, L, dtype=np.int32)

    def leg(threads):
        reps, t = 0, 0.0
        while t < budget_s or reps == 0:
            t0 = time.perf_counter()
            oracle.decode_ragged(q, kc, vc, offs, lens, z, nthreads=threads)
            t += time.perf_counter() - t0
            reps += 1
        return decode_bytes(H, KV, [L] * nseq) * reps / t / 1e9, reps, t

    host = host_info()
    threads = max(1, min(16, host["nproc"]))
    gbs, reps, t = leg(threads)
    gbs1, reps1, t1 = leg(1)
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{nseq} of the 32 sequences x {reps} reps ({t:.1f} s): oracle in shader order "
                      f"(oracle/bn_oracle.c, -O2, no fast-math), OpenMP {threads} threads",
            "single_core": {"value": round(gbs1, 3), "unit": "GB/s", "cores": 1,
                            "sample": f"the same sample x {reps1} reps ({t1:.1f} s), one thread"},
            "host": host}


ALL = ("decode_8k_batch32", "prefill_4k", "ragged_32", "verify_8", "decode_1k", "prefill_prefix",
       "decode_8k_batch32_rotated", "prefill_4k_rotated", "prefill_4k_f32q", "verify_8_rotated", "prep_4k",
       "prep_decode",
       "gate_rotate_4k", "verify_8k_4b", "verify_16_8k_4b", "layer_decode_8k", "layer_verify_8", "layer_prefill_4k", "kv_copy_8x4k",
       "qkv_decode_4b", "qkv_verify_8_4b", "qkv_prefill_4k_4b", "o_proj_decode_4b", "o_proj_prefill_4k_4b",
       "block_decode_8k_4b", "block_verify_8_4b", "block_prefill_4k_4b")
# ternary projections of the 4B layer (hidden 2560, 16 q heads, 4 kv heads): q_proj 8192 rows (q and gate halves),
# k_proj and v_proj 1024 rows each, all over the 2560-wide normed input; o_proj 2560 rows over the 4096-wide
# rotated attention output, added into the residual
TERNARY = {
    "qkv_decode_4b": dict(T=1, K=2560, os=(8192, 1024, 1024)),
    "qkv_verify_8_4b": dict(T=8, K=2560, os=(8192, 1024, 1024)),
    "qkv_prefill_4k_4b": dict(T=4096, K=2560, os=(8192, 1024, 1024)),
    "o_proj_decode_4b": dict(T=1, K=4096, os=(2560,), add=True),
    "o_proj_prefill_4k_4b": dict(T=4096, K=4096, os=(2560,), add=True),
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default=",".join(ALL), help="comma-separated workloads to run")
    ap.add_argument("--copy-calib", type=int, default=0, help="MiB of plain device copy to run first")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the attention path has no cross-GPU exchange); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    only = [w for w in args.only.split(",") if w]
    import torch
    ba = load_package().bonsai_attn
    ctx = ba.Context(0)
    W = Workloads(torch, ba, ctx)
    log = lambda s: print("bench: " + s, file=sys.stderr, flush=True)
    if args.copy_calib:
        log(f"copy calibration {args.copy_calib} MiB x3")
        copy_calibration(torch, args.copy_calib)
    K, Wm = args.steps, args.warmup
    res = {}
    if "decode_8k_batch32" in only:
        log(f"decode_8k_batch32 steps={K} warmup={Wm}")
        res["decode_8k_batch32"] = r = W.decode_batch(K, Wm)
        log(f"  {r['gbs']:.1f} GB/s ({r['ms'] * 1e3:.1f} us/step)")
    if "prefill_4k" in only:
        log("prefill_4k")
        res["prefill_4k"] = r = W.attn(K, Wm, 16, 4, 4096, 0, ba.KIND_PREFILL,
                                       0xB0A5A103, q_f16=True)
        r["steps"], r["warmup"] = K, Wm
        log(f"  {r['tflops']:.1f} TFLOP/s ({r['ms']:.3f} ms/step)")
    if "ragged_32" in only:
        lens = ragged_lengths()
        log(f"ragged_32 (sum of lengths {sum(lens)})")
        res["ragged_32"] = r = W.decode_batch(K, Wm, lens=lens, seed=0xB0A5A105)
        r["sum_len"] = sum(lens)
        log(f"  {r['gbs']:.1f} GB/s ({r['ms'] * 1e3:.1f} us/step)")
    if "verify_8" in only:
        log("verify_8")
        res["verify_8"] = r = W.attn(K, Wm, 8, 2, 8, 2048, ba.KIND_VERIFY, 0xB0A5A102)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "verify_8k_4b" in only:
        log("verify_8k_4b (8 rows over 8184 cached rows, 16/4 heads)")
        res["verify_8k_4b"] = r = W.attn(K, Wm, 16, 4, 8, 8184, ba.KIND_VERIFY, 0xB0A5A10A)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "verify_16_8k_4b" in only:
        log("verify_16_8k_4b (16 rows, the reference's largest verify, over 8176 cached rows, 16/4 heads)")
        res["verify_16_8k_4b"] = r = W.attn(K, Wm, 16, 4, 16, 8176, ba.KIND_VERIFY, 0xB0A5A10B)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "decode_1k" in only:
        log("decode_1k")
        res["decode_1k"] = r = W.attn(K, Wm, 8, 2, 1, 1023, ba.KIND_DECODE, 0xB0A5A100)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "prefill_prefix" in only:
        log("prefill_prefix")
        res["prefill_prefix"] = r = W.attn(K, Wm, 8, 2, 256, 512, ba.KIND_PREFILL, 0xB0A5A101)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['tflops']:.2f} TFLOP/s")
    if "decode_8k_batch32_rotated" in only:
        log("decode_8k_batch32_rotated")
        res["decode_8k_batch32_rotated"] = r = W.decode_batch(K, Wm, rotate=True)
        log(f"  {r['gbs']:.1f} GB/s ({r['ms'] * 1e3:.1f} us/step)")
    if "prefill_4k_rotated" in only:
        log("prefill_4k_rotated")
        res["prefill_4k_rotated"] = r = W.attn(K, Wm, 16, 4, 4096, 0, ba.KIND_PREFILL,
                                               0xB0A5A103, q_f16=True, rotate=True)
        log(f"  {r['tflops']:.1f} TFLOP/s ({r['ms']:.3f} ms/step)")
    if "prefill_4k_f32q" in only:
        log("prefill_4k_f32q (fp32 q: the reference's precision, fp16 hi/lo pair on prefill_hilo_kernel)")
        res["prefill_4k_f32q"] = r = W.attn(K, Wm, 16, 4, 4096, 0, ba.KIND_PREFILL,
                                            0xB0A5A103, q_f16=False)
        log(f"  {r['tflops']:.1f} TFLOP/s ({r['ms']:.3f} ms/step)")
    if "verify_8_rotated" in only:
        log("verify_8_rotated")
        res["verify_8_rotated"] = r = W.attn(K, Wm, 8, 2, 8, 2048, ba.KIND_VERIFY, 0xB0A5A102, rotate=True)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "prep_4k" in only:
        log("prep_4k")
        res["prep_4k"] = r = W.prep(K, Wm, 16, 4, 4096, 0)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "prep_decode" in only:
        log("prep_decode")
        res["prep_decode"] = r = W.prep(K, Wm, 16, 4, 1, 8191)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "gate_rotate_4k" in only:
        log("gate_rotate_4k")
        res["gate_rotate_4k"] = r = W.rotate(K, Wm, 16, 4096)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "layer_decode_8k" in only:
        log("layer_decode_8k")
        res["layer_decode_8k"] = r = W.layer(K, Wm, 16, 4, 1, 8191)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "layer_verify_8" in only:
        log("layer_verify_8")
        res["layer_verify_8"] = r = W.layer(K, Wm, 16, 4, 8, 8184)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    if "layer_prefill_4k" in only:
        log("layer_prefill_4k")
        res["layer_prefill_4k"] = r = W.layer(K, Wm, 16, 4, 4096, 0)
        log(f"  {r['tflops']:.1f} TFLOP/s ({r['ms']:.3f} ms/step)")
    if "kv_copy_8x4k" in only:
        log("kv_copy_8x4k")
        res["kv_copy_8x4k"] = r = W.kv_copy(K, Wm, 8, 4, 4096, 8192)
        log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s")
    for name, cfg in TERNARY.items():
        if name in only:
            log(name)
            res[name] = r = W.ternary(K, Wm, **cfg)
            log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s, {r['tflops']:.1f} TFLOP/s")
    for name, (T, off) in {"block_decode_8k_4b": (1, 8191), "block_verify_8_4b": (8, 8184),
                           "block_prefill_4k_4b": (4096, 0)}.items():
        if name in only:
            log(name)
            res[name] = r = W.block(K, Wm, T, off)
            log(f"  {r['ms'] * 1e3:.1f} us/step, {r['gbs']:.1f} GB/s, {r['tflops']:.1f} TFLOP/s")
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline()
    head = res.get("decode_8k_batch32")
    line = {
        "metric": "attn decode GB/s (%HBM peak) @8K KV; prefill TFLOP/s (%MFMA peak)",
        "value": round(head["gbs"], 2) if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": Wm,
        "ms_per_step": round(head["ms"], 5) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV, f32 accumulate",
        "data": "synthetic (seeded: RMS-normalised N(0,1) q/k rows, N(0,1) v and gate logits)",
        "config": {"workload": "decode_8k_batch32", "sequences": 32, "q_heads": 16, "kv_heads": 4,
                   "head_dim": 256, "kv_rows_per_sequence": 8192, "kv_dtype": "fp16", "append": True,
                   "gate": True},
        "roofline": None,
        "cpu_baseline": cpu,
    }
    if head:
        traffic, src = measured_traffic("decode_8k_batch32_hbm_traffic.md")
        line["roofline"] = {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                            "traffic_source": src,
                            "kernel": "bn::decode_split_kernel<2, false> + bn::decode_combine_kernel (one library call, "
                                      "timed as a whole; profiles/attn_kernels_all_workloads_trace.md has each)",
                            "algorithmic_bytes": head["bytes"]}
    pre = res.get("prefill_4k")
    if pre:
        line["prefill"] = {"workload": "prefill_4k", "value": round(pre["tflops"], 3), "unit": "TFLOP/s",
                           "ms_per_step": round(pre["ms"], 5), "steps": pre["steps"], "warmup": pre["warmup"],
                           "flops": pre["flops"], "peak": MFMA_F16_PEAK_TFLOPS,
                           "frac": round(pre["tflops"] / MFMA_F16_PEAK_TFLOPS, 5)}
    others = {}
    for name in ALL[2:]:
        r = res.get(name)
        if r:
            o = {"us_per_step": round(r["ms"] * 1e3, 3), "GB/s": round(r["gbs"], 2),
                 "hbm_frac": round(r["gbs"] / HBM_PEAK_GBS, 4), "bytes": r["bytes"]}
            if "tflops" in r:
                o["TFLOP/s"] = round(r["tflops"], 3)
                o["mfma_frac"] = round(r["tflops"] / MFMA_F16_PEAK_TFLOPS, 5)
            if "sum_len" in r:
                o["sum_len"] = r["sum_len"]
            others[name] = o
    if others:
        line["workloads"] = others
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
