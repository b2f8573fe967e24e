"""Parity of the HIP path with the oracle on the exact inputs the benchmark times, and at peaky score scales.

The benchmarked workloads are drawn on the GPU by bench.py's own input functions (the same seeds and shapes), copied
to the host, and every output row is compared with the oracle (max-abs 2e-3, projected argmax; rows whose two best
projected reference values tie within the margin that the oracle with fp16-rounded probabilities sets are not
compared, at most max(2, rows / 100) of them). Cache rows written by the call are compared
bit for bit.
  - decode_8k_batch32: 32 sequences x 8192 fp16 KV rows, 16 query / 4 kv heads, append + gate (the headline);
  - ragged_32: 32 sequences with lengths from random.Random(0xB0A5A104) in [1024, 32768] (sum 507,255);
  - prefill_4k: all 4096 rows of the causal prefill, 16/4 heads, with fp16 q (BN_Q_F16; prefill_kernel and
    prefill_pair_kernel) and with fp32 q (prefill_hilo_kernel).
The peaky cases multiply the RMS-normalised q and k rows by a norm weight w (scores q.k/16 then have standard
deviation w^2: tens at w = 4..8), where rounding q to fp16 in an MFMA kernel would move a score by about 1e-4 w^2.
"""
import numpy as np
import pytest

import bench
import oracle
import workload
from conftest import context_with
from glimpse_language_amd import bonsai_attn as ba
from test_gpu_attn import assert_parity, cache_np

pytestmark = pytest.mark.gpu


def host(t):
    return t.cpu().numpy()


def ragged_case(gpu, lens, seed):
    torch, ctx, ws = gpu
    H, KV, nseq = 16, 4, len(lens)
    x = bench.decode_batch_inputs(torch, lens, H, KV, seed)
    print(f"ragged parity: {nseq} sequences, sum of lengths {sum(lens)}, seed {seed:#x}", flush=True)
    kc0, vc0 = host(x["kc"]).view(np.uint16), host(x["vc"]).view(np.uint16)
    q, k_new, v_new, z = host(x["q"]), host(x["k_new"]), host(x["v_new"]), host(x["gate"])
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    lens_np = np.asarray(lens, dtype=np.int32)
    out = ba.decode_ragged(ctx, ws, x["q"], x["kc"], x["vc"], x["kv_off"], x["kv_len"], max(lens), k_new=x["k_new"],
                           v_new=x["v_new"], gate=x["gate"])
    torch.cuda.synchronize()
    last = offs + lens_np - 1  # the appended row of every sequence
    kc_ref, vc_ref = kc0.copy(), vc0.copy()
    kc_ref[last] = oracle.f32_to_f16(k_new)
    vc_ref[last] = oracle.f32_to_f16(v_new)
    ref = oracle.decode_ragged(q, kc_ref, vc_ref, offs, lens_np, z)
    ref16 = oracle.decode_ragged(q, kc_ref, vc_ref, offs, lens_np, z, p16=True)
    err = assert_parity(host(out), ref, H, f"ragged {nseq} seqs", ref16)
    kc1, vc1 = cache_np(x["kc"]), cache_np(x["vc"])
    assert np.array_equal(kc1[last], kc_ref[last]) and np.array_equal(vc1[last], vc_ref[last]), "appended rows"
    # every other row is untouched: compare in slices to bound host memory
    for a, b in ((kc1, kc_ref), (vc1, vc_ref)):
        for r0 in range(0, a.shape[0], 1 << 16):
            assert np.array_equal(a[r0:r0 + (1 << 16)], b[r0:r0 + (1 << 16)]), f"cache rows from {r0}"
    print(f"ragged parity: max-abs {err:.3e}", flush=True)


def test_headline_decode_8k_batch32(gpu):
    ragged_case(gpu, [8192] * 32, 0xB0A5A104)


def test_ragged_32_as_benchmarked(gpu):
    lens = bench.ragged_lengths()
    assert sum(lens) == 507255 and len(lens) == 32
    ragged_case(gpu, lens, 0xB0A5A105)


def prefill_4k_case(gpu, q_f16, ctx=None):
    torch, ctx0, ws0 = gpu
    ctx = ctx or ctx0
    ws = ws0 if ctx is ctx0 else ba.Workspace(ctx, "cuda")
    H, KV, T, off = 16, 4, 4096, 0
    x = bench.attn_inputs(torch, H, KV, T, off, 0xB0A5A103, q_f16=q_f16)
    print(f"prefill_4k parity: 4096 rows, 16/4 heads, {'fp16' if q_f16 else 'fp32'} q", flush=True)
    kc0, vc0 = host(x["kc"]).view(np.uint16).copy(), host(x["vc"]).view(np.uint16).copy()
    out = ba.attention(ctx, ws, x["q"], x["kc"], x["vc"], off, k_new=x["k_new"], v_new=x["v_new"], gate=x["gate"],
                       kind=ba.KIND_PREFILL)
    torch.cuda.synchronize()
    oracle.append(host(x["k_new"]), host(x["v_new"]), kc0, vc0, off)
    q32 = host(x["q"].float())  # the q the kernel read, exactly
    ref = oracle.attend(q32, kc0, vc0, off, host(x["gate"]))
    ref16 = oracle.attend(q32, kc0, vc0, off, host(x["gate"]), p16=True)
    err = assert_parity(host(out), ref, H, "prefill_4k", ref16)
    assert np.array_equal(cache_np(x["kc"]), kc0) and np.array_equal(cache_np(x["vc"]), vc0)
    print(f"prefill_4k parity: max-abs {err:.3e}", flush=True)


def test_prefill_4k_all_rows_fp16_q(gpu):
    prefill_4k_case(gpu, True)


def test_prefill_4k_all_rows_fp16_q_pair_kernel(gpu):
    """The same rows on prefill_pair_kernel (BONSAI_ATTN_PREFILL_PAIR=1)."""
    ctx = context_with(BONSAI_ATTN_PREFILL_PAIR=1)
    try:
        prefill_4k_case(gpu, True, ctx)
    finally:
        gpu[0].cuda.synchronize()
        ctx.close()


def test_prefill_4k_all_rows_fp32_q(gpu):
    """All 4096 rows with fp32 q (the reference's precision; prefill_hilo_kernel multiplies q as fp16 hi + lo)."""
    prefill_4k_case(gpu, False)


def peaky(seed, T, off, H, KV, w):
    """workload.layer with q, k cache rows and new k rows scaled by w (k rows rounded to fp16 after scaling)."""
    inp = workload.layer(seed, T=T, off=off, H=H, KV=KV)
    inp["q"] = (inp["q"] * w).astype(np.float32)
    k = oracle.rms_rows(oracle.normal(seed, 2, (inp["cap"], KV, 256))) * w
    inp["kc"] = oracle.f32_to_f16(k.astype(np.float32))
    inp["k_new"] = (inp["k_new"] * w).astype(np.float32)
    return inp


def to_dev(torch, inp):
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return dict(q=t(inp["q"]), k_new=t(inp["k_new"]), v_new=t(inp["v_new"]), gate=t(inp["gate"]),
                kc=t(inp["kc"].view(np.int16)), vc=t(inp["vc"].view(np.int16)))


@pytest.mark.parametrize("w", [2.0, 4.0, 8.0])
@pytest.mark.parametrize("T,off,H,KV", [(8, 2048, 8, 2), (8, 8184, 16, 4), (4, 300, 8, 2)])
def test_verify_peaky_scores(gpu, w, T, off, H, KV):
    """Verify rows at peaky scores: within 2e-3 of the oracle (argmax equal), and each row within 2e-4 of a
    decode of that row (the equivalence speculative accept relies on)."""
    torch, ctx, ws = gpu
    inp = peaky(0x9E00 + T + off, T, off, H, KV, w)
    d = to_dev(torch, inp)
    out = ba.attention(ctx, ws, d["q"], d["kc"], d["vc"], off, k_new=d["k_new"], v_new=d["v_new"], gate=d["gate"],
                       kind=ba.KIND_VERIFY)
    torch.cuda.synchronize()
    ref, _, _ = workload.expected(inp)
    assert_parity(host(out), ref, H, f"verify w={w}", workload.expected(inp, p16=True)[0])
    for t in range(T):
        o = ba.attention(ctx, ws, d["q"][t:t + 1], d["kc"], d["vc"], off + t, gate=d["gate"][t:t + 1],
                         kind=ba.KIND_DECODE)
        torch.cuda.synchronize()
        diff = float(np.max(np.abs(host(o)[0] - host(out)[t])))
        assert diff <= 2e-4, f"row {t}: verify and decode differ by {diff:.3e}"


@pytest.mark.parametrize("q16,path", [(True, "flash"), (False, "flash"), (True, "prefill"), (False, "prefill")])
@pytest.mark.parametrize("w", [2.0, 4.0, 8.0])
@pytest.mark.parametrize("T,off,H,KV", [(256, 512, 8, 2), (512, 0, 16, 4)])
def test_prefill_peaky_scores(gpu, w, T, off, H, KV, q16, path):
    """Prefill rows at peaky scores: within 2e-3 of the oracle, argmax equal. With q16 the query rows are given as
    fp16 (BN_Q_F16, the oracle sees the same fp16 values); otherwise as fp32, which flash_kernel<true> and
    prefill_hilo_kernel multiply as fp16 hi + lo parts. path "prefill" lowers the block threshold so these shapes run
    on the prefill kernels (prefill_kernel for fp16 q, prefill_hilo_kernel for fp32 q) instead of flash_kernel."""
    torch = gpu[0]
    if path == "prefill":
        ctx = context_with(BONSAI_ATTN_PREFILL_MIN_BLOCKS=1)
        ws = ba.Workspace(ctx, "cuda")
    else:
        _, ctx, ws = gpu
    inp = peaky(0x9F00 + T + off, T, off, H, KV, w)
    if q16:
        inp["q"] = inp["q"].astype(np.float16).astype(np.float32)
    d = to_dev(torch, inp)
    q = d["q"].half() if q16 else d["q"]
    print(f"prefill peaky: T={T} off={off} w={w} q16={q16} path={path}", flush=True)
    out = ba.attention(ctx, ws, q, d["kc"], d["vc"], off, k_new=d["k_new"], v_new=d["v_new"], gate=d["gate"],
                       kind=ba.KIND_PREFILL)
    torch.cuda.synchronize()
    ref, _, _ = workload.expected(inp)
    assert_parity(host(out), ref, H, f"prefill w={w}", workload.expected(inp, p16=True)[0])
    if path == "prefill":
        ctx.close()
