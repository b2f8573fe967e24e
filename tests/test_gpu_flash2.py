"""Parity of flash2_kernel (64 query rows per wave, T >= 64) with the oracle, on the GPU.

By default the library sends a T >= 64 call to flash2_kernel only when it gives at least 128 q-tile blocks (for
example the 4096-row prefill); here a second context created with BONSAI_ATTN_FLASH2_MIN_BLOCKS=1 sends every
T >= 64 call there, so small shapes cover its tails, offsets, head counts and its restart path.
"""
import os

import numpy as np
import pytest

import oracle
import workload
from test_gpu_attn import assert_parity, cache_np, to_dev
from glimpse_language_amd import bonsai_attn as ba

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def f2(gpu):
    torch, _, _ = gpu
    old = os.environ.get("BONSAI_ATTN_FLASH2_MIN_BLOCKS")
    os.environ["BONSAI_ATTN_FLASH2_MIN_BLOCKS"] = "1"
    try:
        ctx = ba.Context(0)
    finally:
        if old is None:
            del os.environ["BONSAI_ATTN_FLASH2_MIN_BLOCKS"]
        else:
            os.environ["BONSAI_ATTN_FLASH2_MIN_BLOCKS"] = old
    ws = ba.Workspace(ctx, "cuda")
    yield torch, ctx, ws
    torch.cuda.synchronize()
    ctx.close()


def run_case(f2, inp, q16=False):
    torch, ctx, ws = f2
    d = to_dev(torch, inp)
    q = d["q"].half() if q16 else d["q"]
    out = ba.attention(ctx, ws, q, d["kc"], d["vc"], inp["off"], k_new=d["k_new"], v_new=d["v_new"],
                       gate=d["gate"], kind=ba.KIND_PREFILL)
    torch.cuda.synchronize()
    return out.cpu().numpy(), d


@pytest.mark.parametrize("T,off,H,KV,gate", [(64, 0, 4, 1, True), (100, 37, 8, 2, True), (130, 500, 16, 4, False),
                                             (200, 0, 8, 2, True), (65, 63, 4, 1, True), (256, 512, 8, 2, True)])
def test_flash2_shapes(f2, T, off, H, KV, gate):
    inp = workload.layer(5000 + T + off, T=T, off=off, H=H, KV=KV, gate=gate)
    out, d = run_case(f2, inp)
    ref, kc_ref, vc_ref = workload.expected(inp)
    assert_parity(out, ref, H, f"flash2 T={T} off={off}")
    assert np.array_equal(cache_np(d["kc"]), kc_ref)
    assert np.array_equal(cache_np(d["vc"]), vc_ref)
    out2, _ = run_case(f2, inp)
    assert np.array_equal(out, out2), "repeat run not bit-identical"


def test_flash2_fp16_q(f2):
    inp = workload.layer(5100, T=96, off=40, H=8, KV=2)
    inp["q"] = inp["q"].astype(np.float16).astype(np.float32)  # values the fp16 path carries exactly
    out, _ = run_case(f2, inp, q16=True)
    ref, _, _ = workload.expected(inp)
    assert_parity(out, ref, 8, "flash2 fp16 q")


def test_flash2_restart_on_late_dominant_key(f2):
    """A key far above the first tile's scores (log2 growth > 14) forces the block to restart; the row then
    returns that key's V row."""
    inp = workload.layer(5200, T=70, off=300, H=4, KV=1, gate=False)
    kc = inp["kc"]
    j = 250
    kj = oracle.f16_to_f32(kc[j, 0])
    inp["q"][50, 2] = 8.0 * kj  # score of key j for row 50, head 2: 8*|k_j|^2/16 = 128 (185 in log2 units)
    out, _ = run_case(f2, inp)
    ref, _, vc_ref = workload.expected(inp)
    assert_parity(out, ref, 4, "flash2 restart")
    assert np.max(np.abs(out[50, 2] - oracle.f16_to_f32(vc_ref[j, 0]))) < 2e-3


def test_flash2_matches_default_path(f2, gpu):
    """The two kernel families agree (each is within 2e-3 of the oracle; here they are compared directly)."""
    torch, ctx1, ws1 = gpu
    inp = workload.layer(5300, T=160, off=96, H=8, KV=2)
    out2, _ = run_case(f2, inp)
    d = to_dev(torch, inp)
    out1 = ba.attention(ctx1, ws1, d["q"], d["kc"], d["vc"], inp["off"], k_new=d["k_new"], v_new=d["v_new"],
                        gate=d["gate"], kind=ba.KIND_PREFILL)
    torch.cuda.synchronize()
    assert np.max(np.abs(out1.cpu().numpy() - out2)) < 1e-3
