"""Parity of the long-prefill kernels with the oracle: prefill_kernel (fp16 q; 8 waves per block, key range
split between two wave groups), prefill_pair_kernel (fp16 q; 4 waves per block, two query heads per wave; chosen with
BONSAI_ATTN_PREFILL_PAIR=1) and prefill_hilo_kernel (fp32 q as an fp16 hi/lo pair; one wave per SIMD, 4-stage copy
ring). Every test runs once per fp16-q kernel.

By default the library sends a T >= 2 call to these kernels only when it gives at least as many 32-token q-tile
blocks as the GPU has CUs (for example the 4096-row prefill); here a second context created with
BONSAI_ATTN_PREFILL_MIN_BLOCKS=1 sends every T >= 2 call there, so small shapes cover their tails, offsets,
head counts, prefill_kernel's merge of an empty or partly empty second half, and the rescale path. Every case
runs with fp16 q (query rows rounded to fp16 first, so the oracle sees the values the kernel multiplies) and with
fp32 q.
"""
import numpy as np
import pytest

import oracle
import workload
from conftest import context_with
from test_gpu_attn import assert_parity, cache_np, to_dev
from glimpse_language_amd import bonsai_attn as ba

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["prefill_kernel", "prefill_pair_kernel"])
def pf(gpu, request):
    """A context that sends every T >= 2 call to the prefill kernels; fp16-q calls on the kernel named by the param
    (BONSAI_ATTN_PREFILL_PAIR), fp32-q calls on prefill_hilo_kernel either way."""
    torch, _, _ = gpu
    print(f"prefill kernel for fp16 q: {request.param}", flush=True)
    ctx = context_with(BONSAI_ATTN_PREFILL_MIN_BLOCKS=1,
                       BONSAI_ATTN_PREFILL_PAIR=int(request.param == "prefill_pair_kernel"))
    ws = ba.Workspace(ctx, "cuda")
    yield torch, ctx, ws
    torch.cuda.synchronize()
    ctx.close()


def run_case(pf, inp, q16=False, dev=None, append=True):
    torch, ctx, ws = pf
    d = dev or to_dev(torch, inp)
    q = d["q"].half() if q16 else d["q"]
    out = ba.attention(ctx, ws, q, d["kc"], d["vc"], inp["off"], k_new=d["k_new"] if append else None,
                       v_new=d["v_new"] if append else None, gate=d["gate"], kind=ba.KIND_PREFILL)
    torch.cuda.synchronize()
    return out.cpu().numpy(), d


SHAPES = workload.PREFILL_SHAPES


def fp16_exact(inp):
    inp["q"] = inp["q"].astype(np.float16).astype(np.float32)
    return inp


@pytest.mark.parametrize("q16", [True, False])
@pytest.mark.parametrize("T,off,H,KV,gate", SHAPES)
def test_prefill_kernel_shapes(pf, T, off, H, KV, gate, q16):
    inp = workload.prefill_shape_input(T, off, H, KV, gate, q16)
    print(f"prefill shapes: T={T} off={off} H={H} KV={KV} fp16 q {q16}", flush=True)
    out, d = run_case(pf, inp, q16=q16)
    ref, kc_ref, vc_ref = workload.expected(inp)
    assert_parity(out, ref, H, f"prefill T={T} off={off} H={H} q16={q16}", workload.expected(inp, p16=True)[0])
    assert np.array_equal(cache_np(d["kc"]), kc_ref)
    assert np.array_equal(cache_np(d["vc"]), vc_ref)
    out2, _ = run_case(pf, inp, q16=q16, dev=d, append=False)
    assert np.array_equal(out, out2), "repeat run not bit-identical"


def test_prefill_kernel_fp16_q(pf):
    inp = workload.layer(6100, T=96, off=40, H=8, KV=2)
    inp["q"] = inp["q"].astype(np.float16).astype(np.float32)  # values the fp16 path carries exactly
    out, _ = run_case(pf, inp, q16=True)
    ref, _, _ = workload.expected(inp)
    assert_parity(out, ref, 8, "prefill_kernel fp16 q", workload.expected(inp, p16=True)[0])


@pytest.mark.parametrize("q16", [True, False])
def test_prefill_kernel_rescale_on_late_dominant_key(pf, q16):
    """A key far above the earlier scores (log2 growth > 8) moves the running max and rescales O; the row then
    returns that key's V row. Key 250 sits in the first half of the key range of row 50's q-tile (positions
    300..369, 12 key tiles), key 340 in the second half."""
    inp = workload.layer(6200, T=70, off=300, H=4, KV=1, gate=False)
    kc = inp["kc"]
    for row, head, j in ((50, 2, 250), (60, 1, 290)):
        kj = oracle.f16_to_f32(kc[j, 0])
        inp["q"][row, head] = 8.0 * kj  # score of key j: 8*|k_j|^2/16 = 128 (185 in log2 units)
    if q16:
        fp16_exact(inp)  # 8 k_j is exact in fp16
    out, _ = run_case(pf, inp, q16=q16)
    ref, _, vc_ref = workload.expected(inp)
    assert_parity(out, ref, 4, "prefill_kernel rescale", workload.expected(inp, p16=True)[0])
    assert np.max(np.abs(out[50, 2] - oracle.f16_to_f32(vc_ref[250, 0]))) < 2e-3
    assert np.max(np.abs(out[60, 1] - oracle.f16_to_f32(vc_ref[290, 0]))) < 2e-3


@pytest.mark.parametrize("q16", [True, False])
def test_prefill_kernel_matches_default_path(pf, gpu, q16):
    """The prefill kernels and flash_kernel agree (each is within 2e-3 of the oracle; here they are compared
    directly)."""
    torch, ctx1, ws1 = gpu
    inp = workload.layer(6300, T=160, off=96, H=8, KV=2)
    if q16:
        fp16_exact(inp)
    out2, _ = run_case(pf, inp, q16=q16)
    d = to_dev(torch, inp)
    out1 = ba.attention(ctx1, ws1, d["q"].half() if q16 else d["q"], d["kc"], d["vc"], inp["off"], k_new=d["k_new"],
                        v_new=d["v_new"], gate=d["gate"], kind=ba.KIND_PREFILL)
    torch.cuda.synchronize()
    assert np.max(np.abs(out1.cpu().numpy() - out2)) < 1e-3


@pytest.mark.parametrize("q16", [True, False])
def test_prefill_q_and_gate_in_place_from_qproj(pf, q16):
    """q read in place from the first half of a [T][H][512] q_proj-shaped buffer (q_ts = 512 H, q_hs = 512 elements)
    and the gate from its second half, the layout the runtime's q projection writes: the strided Q copies into LDS
    (fp16 q) and loads (fp32 q) give the packed layout's outputs bit for bit."""
    torch, ctx, ws = pf
    T, off, H, KV = 100, 37, 8, 2
    inp = workload.layer(6400, T=T, off=off, H=H, KV=KV)
    if q16:
        fp16_exact(inp)
    print(f"prefill q and gate in place: T={T} off={off} fp16 q {q16}", flush=True)
    packed, d = run_case(pf, inp, q16=q16)
    qp = torch.zeros((T, H, 512), dtype=torch.float32, device="cuda")
    qp[:, :, :256] = d["q"]
    qp[:, :, 256:] = d["gate"]
    qsrc = qp.half() if q16 else qp
    out = ba.attention(ctx, ws, qsrc[:, :, :256], d["kc"], d["vc"], off, gate=qp[:, :, 256:],
                       q_strides=(512 * H, 512), g_strides=(512 * H, 512), kind=ba.KIND_PREFILL)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), packed), "strided q / gate differ from the packed layout"
