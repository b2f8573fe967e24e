"""The device-side cache offset (bn_attn_args.dyn / bn_prep_args.dyn, the reference's dynamic parameter slot for
replayed command buffers: attn_split.comp:12-14, attn_prep.comp:32-33, gpu_vk.rs:1035-1049) on the GPU.

1. A decode step of the whole attention arm (bn_attn_layer, T = 1: norm, mRoPE, fp16 append, attention, gate,
   rotation) is captured once in a HIP graph together with a device-side increment of the offset and of the mRoPE
   positions, then replayed for 8 consecutive tokens. Before each replay the caller writes that token's raw
   projection rows into the captured input buffers. Every replay is checked against the oracle's chain for that
   token (max-abs 2e-3, projected argmax), and the cache rows written by the replays against the oracle's (K within
   one fp16 ulp, V exact; every other row untouched).
2. Every kernel path (decode, verify rows on the MFMA kernel, rows as decodes, the three prefill kernels, the append)
   called with a device offset below the host bound gives the oracle's result at the device offset, and writes the
   cache rows at the device offset.
3. The same for the one-call layer (bn_attn_layer) past one row, where prep_kernel reads the device offset too:
   verify rows, rows as decodes, and prefills, against the oracle's chain at the device offset.
"""
import ctypes

import numpy as np
import pytest

import oracle
import workload
from conftest import context_with
from test_gpu_attn import assert_parity, cache_np
from test_gpu_prep_rotate import inv_freq, oracle_prep, prep_inputs, to_dev
from test_gpu_layer import assert_k_close
from glimpse_language_amd import bonsai_attn as ba

pytestmark = pytest.mark.gpu
D = 256


def test_decode_layer_graph_replay(gpu):
    torch, ctx, ws = gpu
    H, KV, off0, steps, cap = 16, 4, 2000, 8, 2100
    seed = 0x6A00
    qp = oracle.normal(seed, 0, (steps, 1, H, 512)) * np.float32(2.5)
    kp = oracle.normal(seed, 1, (steps, 1, KV, D)) * np.float32(0.7)
    vp = oracle.normal(seed, 2, (steps, 1, KV, D))
    qn = (1.0 + 0.1 * oracle.normal(seed, 3, (D,))).astype(np.float32)
    kn = (1.0 + 0.1 * oracle.normal(seed, 4, (D,))).astype(np.float32)
    kc0 = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(seed, 5, (cap, KV, D))))
    vc0 = oracle.f32_to_f16(oracle.normal(seed, 6, (cap, KV, D)))
    signs = np.where(oracle.normal(seed, 9, (H * D,)) > 0, 1.0, -1.0).astype(np.float32)
    inv = inv_freq()

    # captured buffers: this token's raw rows, its positions [3][1] and the offset
    qp_s = torch.zeros((1, H, 512), device="cuda")
    kp_s = torch.zeros((1, KV, D), device="cuda")
    vp_s = torch.zeros((1, KV, D), device="cuda")
    pos_s = torch.full((3, 1), off0, dtype=torch.int32, device="cuda")
    dyn_s = torch.full((1,), off0, dtype=torch.int32, device="cuda")
    out = torch.zeros((1, H, D), device="cuda")
    kc, vc = to_dev(torch, kc0), to_dev(torch, vc0)
    qn_d, kn_d, inv_d, signs_d = to_dev(torch, qn), to_dev(torch, kn), to_dev(torch, inv), to_dev(torch, signs)
    # argument blocks (and the workspace) are built before the capture: the call itself allocates nothing
    p, a, out = ba.attention_layer_args(ctx, ws, qp_s, kp_s, vp_s, qn_d, kn_d, pos_s, inv_d, kc, vc, cap - 1,
                                        gate=qp_s[:, :, D:], signs=signs_d, out=out, dyn=dyn_s)
    assert a.off == cap - 1 and a.dyn == dyn_s.data_ptr()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = ctx.lib.bn_attn_layer(ctx.h, ctx._stream(None), ctypes.byref(p), ctypes.byref(a))
        dyn_s.add_(1)
        pos_s.add_(1)
    assert st == ba.BN_OK, ctx.error()
    torch.cuda.synchronize()

    kc_ref, vc_ref = kc0.copy(), vc0.copy()
    R = workload.projection(H)
    for s in range(steps):
        off = off0 + s
        print(f"graph replay: token {s} at offset {off}", flush=True)
        qp_s.copy_(torch.from_numpy(qp[s]))
        kp_s.copy_(torch.from_numpy(kp[s]))
        vp_s.copy_(torch.from_numpy(vp[s]))
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(1, H * D)
        # the oracle's chain for this token on the oracle's cache
        pos = np.full((3, 1), off, dtype=np.int32)
        q_ref = oracle.prep(qp[s], kp[s], vp[s], qn, kn, pos, inv, kc_ref, vc_ref, off)
        attn = oracle.attend(q_ref, kc_ref, vc_ref, off, qp[s][:, :, D:]).reshape(1, H * D)
        attn16 = oracle.attend(q_ref, kc_ref, vc_ref, off, qp[s][:, :, D:], p16=True).reshape(1, H * D)
        qp_inf = np.zeros((1, H, 512), np.float32)
        qp_inf[:, :, D:] = np.inf  # sigmoid = 1: rotate the already-gated row
        ref = oracle.gate_rotate(attn, qp_inf.reshape(1, -1), signs)
        ref16 = oracle.gate_rotate(attn16, qp_inf.reshape(1, -1), signs)
        err = float(np.max(np.abs(got - ref)))
        assert err <= 2e-3, f"token {s}: max-abs {err:.3e}"
        bad, _ = workload.argmax_mismatches(got, ref, R, ref16)
        assert len(bad) == 0, f"token {s}: projected argmax differs"
    assert int(dyn_s.item()) == off0 + steps and int(pos_s[0, 0].item()) == off0 + steps
    kcg, vcg = cache_np(kc), cache_np(vc)
    rows = slice(off0, off0 + steps)
    assert_k_close(kcg[rows], kc_ref[rows])
    assert np.array_equal(vcg[rows], vc_ref[rows])
    assert np.array_equal(kcg[:off0], kc0[:off0]) and np.array_equal(kcg[off0 + steps:], kc0[off0 + steps:])
    assert np.array_equal(vcg[:off0], vc0[:off0]) and np.array_equal(vcg[off0 + steps:], vc0[off0 + steps:])


# (T, off, off_max, H, KV, kind, min prefill blocks, fp16 q): decode (one split and many), verify rows on the MFMA
# kernel, 12 rows as decodes of their rows, prefill on flash_kernel, prefill_hilo_kernel (fp32 q) and prefill_kernel
# (fp16 q)
@pytest.mark.parametrize("T,off,off_max,H,KV,kind,min_blocks,q16", [
    (1, 40, 5000, 8, 2, ba.KIND_DECODE, 0, False),
    (1, 3000, 9000, 16, 4, ba.KIND_DECODE, 0, False),
    (8, 2048, 4000, 8, 2, ba.KIND_VERIFY, 0, False),
    (12, 700, 2000, 8, 2, ba.KIND_VERIFY, 0, False),
    (100, 300, 1000, 8, 2, ba.KIND_PREFILL, 0, False),
    (64, 200, 900, 8, 2, ba.KIND_PREFILL, 1, False),
    (64, 200, 900, 8, 2, ba.KIND_PREFILL, 1, True),
])
def test_device_offset_every_path(gpu, T, off, off_max, H, KV, kind, min_blocks, q16):
    torch = gpu[0]
    if min_blocks:
        ctx = context_with(BONSAI_ATTN_PREFILL_MIN_BLOCKS=min_blocks)
        ws = ba.Workspace(ctx, "cuda")
    else:
        _, ctx, ws = gpu
    cap = off_max + T
    inp = workload.layer(0x6B00 + T + off, T=T, off=off, H=H, KV=KV, cap=cap)
    if q16:
        inp["q"] = inp["q"].astype(np.float16).astype(np.float32)
    print(f"device offset: T={T} off={off} (host bound {off_max}) H={H} KV={KV} fp16 q {q16}", flush=True)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    kc, vc = t(inp["kc"].view(np.int16)), t(inp["vc"].view(np.int16))
    dyn = torch.tensor([off], dtype=torch.int32, device="cuda")
    q = t(inp["q"]).half() if q16 else t(inp["q"])
    out = ba.attention(ctx, ws, q, kc, vc, off_max, k_new=t(inp["k_new"]), v_new=t(inp["v_new"]),
                       gate=t(inp["gate"]), kind=kind, dyn=dyn)
    torch.cuda.synchronize()
    ref, kc_ref, vc_ref = workload.expected(inp)
    assert_parity(out.cpu().numpy(), ref, H, f"dyn T={T}", workload.expected(inp, p16=True)[0])
    assert np.array_equal(cache_np(kc), kc_ref) and np.array_equal(cache_np(vc), vc_ref)
    if min_blocks:
        ctx.close()


# (T, off_max, H, KV, kind, min prefill blocks): a device offset past the host bound on every path that appends
# (decode, verify rows, the append kernel before a prefill, the prefill kernels)
@pytest.mark.parametrize("T,off_max,H,KV,kind,min_blocks", [
    (1, 3000, 16, 4, ba.KIND_DECODE, 0),
    (8, 2048, 8, 2, ba.KIND_VERIFY, 0),
    (100, 300, 8, 2, ba.KIND_PREFILL, 0),
    (64, 200, 8, 2, ba.KIND_PREFILL, 1),
])
def test_device_offset_past_the_bound_is_flagged_and_appends_nothing(gpu, T, off_max, H, KV, kind, min_blocks):
    """dyn[0] above `off` cannot be returned as an error by the kernels: they attend as at `off`, write no cache
    row and set the device's overflow flag, which bn_dyn_overflow reads and clears. A call within the bound after it
    leaves the flag clear."""
    torch = gpu[0]
    if min_blocks:
        ctx = context_with(BONSAI_ATTN_PREFILL_MIN_BLOCKS=min_blocks)
        ws = ba.Workspace(ctx, "cuda")
    else:
        _, ctx, ws = gpu
    assert ctx.dyn_overflow() in (False, True)  # clears what earlier tests left
    inp = workload.layer(0x6E00 + T + off_max, T=T, off=off_max, H=H, KV=KV, cap=off_max + T)
    print(f"device offset past the bound: T={T} bound {off_max} dyn {off_max + 7} kind {kind}", flush=True)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    kc, vc = t(inp["kc"].view(np.int16)), t(inp["vc"].view(np.int16))
    dyn = torch.tensor([off_max + 7], dtype=torch.int32, device="cuda")
    out = ba.attention(ctx, ws, t(inp["q"]), kc, vc, off_max, k_new=t(inp["k_new"]), v_new=t(inp["v_new"]),
                       gate=t(inp["gate"]), kind=kind, dyn=dyn)
    torch.cuda.synchronize()
    assert ctx.dyn_overflow() is True
    assert ctx.dyn_overflow() is False  # read and cleared
    assert np.array_equal(cache_np(kc), inp["kc"]) and np.array_equal(cache_np(vc), inp["vc"]), "cache rows changed"
    assert np.all(np.isfinite(out.cpu().numpy()))
    dyn.fill_(off_max - 3 if T == 1 else 0)
    ba.attention(ctx, ws, t(inp["q"]), kc, vc, off_max, k_new=t(inp["k_new"]), v_new=t(inp["v_new"]),
                 gate=t(inp["gate"]), kind=kind, dyn=dyn)
    torch.cuda.synchronize()
    assert ctx.dyn_overflow() is False
    if min_blocks:
        ctx.close()


def test_layer_device_offset_past_the_bound_appends_nothing(gpu):
    """The one-call layer with dyn[0] past the bound: prep_kernel writes no K/V row and the flag is set."""
    torch, ctx, ws = gpu
    T, off_max, H, KV = 8, 2000, 8, 2
    ctx.dyn_overflow()
    inp = prep_inputs(0x6F00, T, off_max, H, KV)
    print("layer device offset past the bound: T=8 bound 2000 dyn 2009", flush=True)
    dev = {k: to_dev(torch, inp[k]) for k in ("qp", "kp", "vp", "qn", "kn", "pos", "inv", "kc", "vc")}
    dyn = torch.tensor([off_max + 9], dtype=torch.int32, device="cuda")
    ba.attention_layer(ctx, ws, dev["qp"], dev["kp"], dev["vp"], dev["qn"], dev["kn"], dev["pos"], dev["inv"],
                       dev["kc"], dev["vc"], off_max, gate=dev["qp"][:, :, D:], dyn=dyn)
    torch.cuda.synchronize()
    assert ctx.dyn_overflow() is True
    assert np.array_equal(cache_np(dev["kc"]), inp["kc"]) and np.array_equal(cache_np(dev["vc"]), inp["vc"])


# (T, off, off_max, H, KV, rotate, min prefill blocks): the one-call layer (bn_attn_layer) with a device offset below
# the host bound on its paths past one row: 8 verify rows (prep_kernel<8, 3> writes q and the K/V rows, then
# verify_kernel and the merge), 12 rows (prep_kernel, then decodes of their rows with q normed in the prologue), a
# prefill on flash_kernel and one on prefill_hilo_kernel (prep_kernel<4, 4> writes the fp32 q scratch)
@pytest.mark.parametrize("T,off,off_max,H,KV,rotate,min_blocks", [
    (8, 2048, 4000, 8, 2, True, 0),
    (12, 700, 2000, 8, 2, False, 0),
    (100, 300, 1000, 8, 2, True, 0),
    (64, 200, 900, 8, 2, False, 1),
])
def test_layer_device_offset(gpu, T, off, off_max, H, KV, rotate, min_blocks):
    torch = gpu[0]
    if min_blocks:
        ctx = context_with(BONSAI_ATTN_PREFILL_MIN_BLOCKS=min_blocks)
        ws = ba.Workspace(ctx, "cuda")
    else:
        _, ctx, ws = gpu
    seed = 0x6D10 + T + off  # inputs whose reference leaves at most max(2, rows / 100) argmax ties
    inp = prep_inputs(seed, T, off, H, KV)
    cap = off_max + T
    extra = cap - inp["kc"].shape[0]
    inp["kc"] = np.concatenate([inp["kc"], oracle.f32_to_f16(oracle.normal(seed, 7, (extra, KV, D)))])
    inp["vc"] = np.concatenate([inp["vc"], oracle.f32_to_f16(oracle.normal(seed, 8, (extra, KV, D)))])
    signs = np.where(oracle.normal(seed, 9, (H * D,)) > 0, 1.0, -1.0).astype(np.float32) if rotate else None
    print(f"layer device offset: T={T} off={off} (host bound {off_max}) H={H} KV={KV} rotate={rotate}", flush=True)
    dev = {k: to_dev(torch, inp[k]) for k in ("qp", "kp", "vp", "qn", "kn", "pos", "inv", "kc", "vc")}
    dyn = torch.tensor([off], dtype=torch.int32, device="cuda")
    out = ba.attention_layer(ctx, ws, dev["qp"], dev["kp"], dev["vp"], dev["qn"], dev["kn"], dev["pos"], dev["inv"],
                             dev["kc"], dev["vc"], off_max, gate=dev["qp"][:, :, D:],
                             signs=None if signs is None else torch.from_numpy(signs).cuda(), dyn=dyn)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(T, H * D)
    q_ref, kc_ref, vc_ref = oracle_prep(inp)
    ref = oracle.attend(q_ref, kc_ref, vc_ref, off, inp["qp"][:, :, D:]).reshape(T, H * D)
    ref16 = oracle.attend(q_ref, kc_ref, vc_ref, off, inp["qp"][:, :, D:], p16=True).reshape(T, H * D)
    if rotate:
        qp_inf = np.zeros((T, H, 512), np.float32)
        qp_inf[:, :, D:] = np.inf  # sigmoid = 1: rotate the already-gated rows
        ref = oracle.gate_rotate(ref, qp_inf.reshape(T, -1), signs)
        ref16 = oracle.gate_rotate(ref16, qp_inf.reshape(T, -1), signs)
    assert_parity(got, ref, H, f"layer dyn T={T}", ref16)
    kc, vc = cache_np(dev["kc"]), cache_np(dev["vc"])
    rows = slice(off, off + T)
    assert_k_close(kc[rows], kc_ref[rows])
    assert np.array_equal(vc[rows], vc_ref[rows])
    assert np.array_equal(kc[:off], inp["kc"][:off]) and np.array_equal(kc[off + T:], inp["kc"][off + T:])
    assert np.array_equal(vc[:off], inp["vc"][:off]) and np.array_equal(vc[off + T:], inp["vc"][off + T:])
    if min_blocks:
        ctx.close()
