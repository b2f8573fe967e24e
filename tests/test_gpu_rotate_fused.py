"""Attention calls with `signs`: `out` is o_proj's input, the gated output rotated as gate_rotate does it
(gate_rotate.comp:18-25), inside the attention call.

Checked two ways on every case:
  - against the separate rotation of the same call's gated output (bn_gate_rotate with gate = NULL): the same fp32
    operations in the same order, so within 1e-6 (normally bit-identical);
  - against the oracle: oracle attention, then oracle gate_rotate with the gate logits set to +inf (sigmoid = 1
    exactly, so the oracle rotates its already-gated output): max-abs 2e-3 and the same projected argmax.
Cases cover each kernel that can finish a row: the decode split kernel (one split), the split merge (many
splits), verify rows, prefill_kernel and prefill_hilo_kernel (in their epilogues), flash_kernel (rotated in place after it) and ragged
batches.
"""
import numpy as np
import pytest

import oracle
import workload
from conftest import context_with
from test_gpu_attn import assert_parity, make_ragged, to_dev
from glimpse_language_amd import bonsai_attn as ba

pytestmark = pytest.mark.gpu
D = 256


def signs_for(H, seed=77):
    return np.where(oracle.normal(seed, 0, (H * D,)) > 0, 1.0, -1.0).astype(np.float32)


def oracle_rotate(gated, signs):
    T, W = gated.shape[0], signs.size
    qp = np.zeros((T, W // D, 512), np.float32)
    qp[:, :, D:] = np.inf
    return oracle.gate_rotate(gated.reshape(T, W), qp.reshape(T, -1), signs)


def check_rotated(g, inp, kind, q16=False):
    """q16: the query rows are rounded to fp16 and given as fp16 (BN_Q_F16)."""
    torch, ctx, ws = g
    T, H, off = inp["T"], inp["H"], inp["off"]
    if q16:
        inp["q"] = inp["q"].astype(np.float16).astype(np.float32)
    signs = signs_for(H)
    d_signs = torch.from_numpy(signs).cuda()
    d = to_dev(torch, inp)
    q = d["q"].half() if q16 else d["q"]
    print(f"rotated T={T} off={off} H={H} kind={kind} fp16 q {q16}", flush=True)
    plain = ba.attention(ctx, ws, q, d["kc"], d["vc"], off, k_new=d["k_new"], v_new=d["v_new"],
                         gate=d["gate"], kind=kind)
    rot = ba.attention(ctx, ws, q, d["kc"], d["vc"], off, k_new=d["k_new"], v_new=d["v_new"],
                       gate=d["gate"], kind=kind, signs=d_signs)
    sep = ba.gate_rotate(ctx, plain.reshape(T, H * D), d_signs)
    torch.cuda.synchronize()
    got = rot.reshape(T, H * D).cpu().numpy()
    assert float(np.max(np.abs(got - sep.cpu().numpy()))) <= 1e-6
    ref, _, _ = workload.expected(inp)
    ref16, _, _ = workload.expected(inp, p16=True)
    assert_parity(got.reshape(T, H, D), oracle_rotate(ref, signs).reshape(T, H, D), H, f"rotated T={T} off={off}",
                  oracle_rotate(ref16, signs).reshape(T, H, D))


@pytest.mark.parametrize("L,H,KV", [(1, 8, 2), (64, 8, 2), (65, 8, 2), (5000, 8, 2), (3000, 16, 4)])
def test_decode_rotated(gpu, L, H, KV):
    check_rotated(gpu, workload.layer(0x9100 + L, T=1, off=L - 1, H=H, KV=KV), ba.KIND_DECODE)


@pytest.mark.parametrize("T,off", [(8, 1000), (16, 3), (2, 0)])
def test_verify_rotated(gpu, T, off):
    check_rotated(gpu, workload.layer(0x9200 + T, T=T, off=off, H=8, KV=2), ba.KIND_VERIFY)


def test_forward_flash_rotated(gpu):
    check_rotated(gpu, workload.layer(0x9300, T=100, off=700, H=8, KV=2), ba.KIND_FORWARD)


@pytest.mark.parametrize("q16", [True, False])  # prefill_kernel, prefill_hilo_kernel
@pytest.mark.parametrize("T,off", [(96, 200), (45, 0)])
def test_prefill_kernel_rotated(gpu, T, off, q16):
    torch = gpu[0]
    ctx = context_with(BONSAI_ATTN_PREFILL_MIN_BLOCKS=1)
    ws = ba.Workspace(ctx, "cuda")
    check_rotated((torch, ctx, ws), workload.layer(0x9400 + T, T=T, off=off, H=8, KV=2), ba.KIND_PREFILL, q16)
    torch.cuda.synchronize()
    ctx.close()


@pytest.mark.parametrize("nseq,lo,hi", [(7, 1, 300), (32, 1024, 4096)])
def test_ragged_rotated(gpu, nseq, lo, hi):
    torch, ctx, ws = gpu
    H, KV = 16, 4
    lens, offs, kc, vc, q, k_new, v_new, z = make_ragged(0x9500 + nseq, nseq, H, KV, lo, hi)
    signs = signs_for(H)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    kc_d, vc_d = t(kc.view(np.int16)), t(vc.view(np.int16))
    args = (ctx, ws, t(q), kc_d, vc_d, t(offs), t(lens), int(lens.max()))
    plain = ba.decode_ragged(*args, k_new=t(k_new), v_new=t(v_new), gate=t(z))
    rot = ba.decode_ragged(*args, k_new=t(k_new), v_new=t(v_new), gate=t(z), signs=t(signs))
    sep = ba.gate_rotate(ctx, plain.reshape(nseq, H * D), t(signs))
    torch.cuda.synchronize()
    got = rot.reshape(nseq, H * D).cpu().numpy()
    assert float(np.max(np.abs(got - sep.cpu().numpy()))) <= 1e-6
    kc_ref, vc_ref = kc.copy(), vc.copy()
    for i in range(nseq):
        r = offs[i] + lens[i] - 1
        kc_ref[r] = k_new[i].astype(np.float16).view(np.uint16)
        vc_ref[r] = v_new[i].astype(np.float16).view(np.uint16)
    ref = oracle.decode_ragged(q, kc_ref, vc_ref, offs, lens, z)
    ref16 = oracle.decode_ragged(q, kc_ref, vc_ref, offs, lens, z, p16=True)
    assert_parity(got.reshape(nseq, H, D), oracle_rotate(ref, signs).reshape(nseq, H, D), H, "ragged rotated",
                  oracle_rotate(ref16, signs).reshape(nseq, H, D))
