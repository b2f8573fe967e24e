"""bn_attn_layer (model.rs:828-893 in one call; attn_prep inside the decode kernel's prologue for T <= 16) on the GPU.

Each case is checked against the same layer run as separate calls (bn_attn_prep, then the attention call, then
bn_gate_rotate when rotated): outputs within 1e-5 and cache rows within one fp16 ulp (the norm and rotation are
the same code, but inlined into another kernel the compiler may contract a product differently); and against
the oracle's chain (oracle prep, oracle attention, oracle gate_rotate): max-abs 2e-3 and the same projected
argmax. Cases cover every path of the call: one decode row (prep fused into the split kernel, which also appends
the new K/V row), verify rows (K/V rows by prep_kernel, q in the split kernel's prologue), and prefills through
prefill_kernel and through flash_kernel (q written by prep_kernel to the caller's scratch, fp32 or fp16).
"""
import numpy as np
import pytest

import oracle
import workload
from conftest import context_with
from test_gpu_prep_rotate import oracle_prep, prep_inputs, to_dev
from glimpse_language_amd import bonsai_attn as ba

pytestmark = pytest.mark.gpu
D = 256


def assert_k_close(got, ref):
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and diff.sum() <= 0.01 * diff.size


def run_layer(g, inp, signs, T, off, H, q16=False):
    torch, ctx, ws = g
    dev = {k: to_dev(torch, inp[k]) for k in ("qp", "kp", "vp", "qn", "kn", "pos", "inv", "kc", "vc")}
    d_signs = None if signs is None else torch.from_numpy(signs).cuda()
    q = torch.empty((T, H, D), dtype=torch.float16, device="cuda") if q16 else None
    out = ba.attention_layer(ctx, ws, dev["qp"], dev["kp"], dev["vp"], dev["qn"], dev["kn"], dev["pos"], dev["inv"],
                             dev["kc"], dev["vc"], off, gate=dev["qp"][:, :, D:], signs=d_signs, q=q)
    torch.cuda.synchronize()
    return out, dev


def run_separate(g, inp, signs, T, off, H):
    torch, ctx, ws = g
    dev = {k: to_dev(torch, inp[k]) for k in ("qp", "kp", "vp", "qn", "kn", "pos", "inv", "kc", "vc")}
    q = ba.attn_prep(ctx, dev["qp"], dev["kp"], dev["vp"], dev["qn"], dev["kn"], dev["pos"], dev["inv"], dev["kc"],
                     dev["vc"], off)
    gate = dev["qp"][:, :, D:]
    attn = ba.attention(ctx, ws, q, dev["kc"], dev["vc"], off, gate=gate, g_strides=(gate.stride(0), gate.stride(1)))
    out = attn if signs is None else ba.gate_rotate(ctx, attn.reshape(T, H * D), torch.from_numpy(signs).cuda())
    torch.cuda.synchronize()
    return out.reshape(T, H, D), dev


def check_layer(g, T, off, H, KV, rotate, seed, q16=False):
    inp = prep_inputs(seed, T, off, H, KV)
    signs = np.where(oracle.normal(seed, 9, (H * D,)) > 0, 1.0, -1.0).astype(np.float32) if rotate else None
    print(f"layer T={T} off={off} H={H} KV={KV} rotate={rotate} q16={q16}", flush=True)
    out, dev = run_layer(g, inp, signs, T, off, H, q16)
    sep, dev2 = run_separate(g, inp, signs, T, off, H)
    got = out.cpu().numpy().reshape(T, H, D)
    # an fp16 q (the prefill scratch with BN_Q_F16) moves the scores by fp16 rounding; fp32 q is the same math
    assert float(np.max(np.abs(got - sep.cpu().numpy()))) <= (1e-3 if q16 else 1e-5)
    kc = dev["kc"].cpu().numpy().view(np.uint16)
    vc = dev["vc"].cpu().numpy().view(np.uint16)
    rows = slice(off, off + T)
    assert_k_close(kc[rows], dev2["kc"].cpu().numpy().view(np.uint16)[rows])
    assert np.array_equal(vc, dev2["vc"].cpu().numpy().view(np.uint16))
    # the oracle's chain
    q_ref, kc_ref, vc_ref = oracle_prep(inp)
    assert_k_close(kc[rows], kc_ref[rows])
    assert np.array_equal(vc[rows], vc_ref[rows])
    attn_ref = oracle.attend(q_ref, kc_ref, vc_ref, off, inp["qp"][:, :, D:])
    ref = attn_ref.reshape(T, H * D)
    ref16 = oracle.attend(q_ref, kc_ref, vc_ref, off, inp["qp"][:, :, D:], p16=True).reshape(T, H * D)
    if rotate:
        qp_inf = np.zeros((T, H, 512), np.float32)
        qp_inf[:, :, D:] = np.inf  # sigmoid = 1: rotate the already-gated rows
        ref = oracle.gate_rotate(ref, qp_inf.reshape(T, -1), signs)
        ref16 = oracle.gate_rotate(ref16, qp_inf.reshape(T, -1), signs)
    err = float(np.max(np.abs(got.reshape(T, H * D) - ref)))
    assert err <= 2e-3, err
    R = oracle.normal(workload.PROJ_SEED, 0, (H * D, 128)).astype(np.float64)
    bad, _ = workload.argmax_mismatches(got.reshape(T, -1), ref, R, ref16)
    assert len(bad) == 0, f"projected argmax differs on rows {bad}"


@pytest.mark.parametrize("T,off,H,KV,rotate", [
    (1, 2047, 8, 2, False),     # a decode step: one split launch (+ merge)
    (1, 40, 8, 2, True),        # one split: the split kernel finishes the row
    (1, 9000, 16, 4, True),     # late position, many splits, rotated in the merge
    (8, 1000, 8, 2, True),      # verify rows
    (16, 3, 8, 2, False),
    (200, 300, 8, 2, True),     # small prefill: flash_kernel reads the q that prep_kernel wrote
])
def test_layer_matches_separate_calls_and_oracle(gpu, T, off, H, KV, rotate):
    check_layer(gpu, T, off, H, KV, rotate, 0xD000 + T + off)


@pytest.mark.parametrize("T,off,rotate,q16", [(96, 200, True, False), (45, 0, False, True), (64, 30, True, True)])
def test_layer_prefill_kernel(gpu, T, off, rotate, q16):
    torch = gpu[0]
    ctx = context_with(BONSAI_ATTN_PREFILL_MIN_BLOCKS=1)
    ws = ba.Workspace(ctx, "cuda")
    check_layer((torch, ctx, ws), T, off, 8, 2, rotate, 0xD100 + T, q16)
    torch.cuda.synchronize()
    ctx.close()


def test_layer_rejects_mixed_args(gpu):
    torch, ctx, ws = gpu
    inp = prep_inputs(0xD200, 2, 10, 8, 2)
    dev = {k: to_dev(torch, inp[k]) for k in ("qp", "kp", "vp", "qn", "kn", "pos", "inv", "kc", "vc")}
    out = torch.empty((2, 8, D), device="cuda")
    p = ba.prep_args(dev["qp"], dev["kp"], dev["vp"], dev["qn"], dev["kn"], dev["pos"], dev["inv"], out, dev["kc"],
                     dev["vc"], 10)
    a = ba.attn_args(2, 10, 8, 2, dev["kc"].shape[0], dev["qp"], dev["kc"], dev["vc"], out)  # q must be NULL
    st = ctx.lib.bn_attn_layer(ctx.h, ctx._stream(None), p, a)
    assert st == ba.BN_EINVAL and "NULL" in ctx.error()
    a = ba.attn_args(2, 11, 8, 2, dev["kc"].shape[0], None, dev["kc"], dev["vc"], out)  # off differs
    st = ctx.lib.bn_attn_layer(ctx.h, ctx._stream(None), p, a)
    assert st == ba.BN_EINVAL and "different" in ctx.error()
