"""GPU parity of the steps either side of attention, through the C ABI, against the oracle.

  - bn_attn_prep (attn_prep.comp:29-59): q within 3e-5 of the oracle (fp32; the norm's sum order and the sin/cos
    routine differ by a few ulp), k cache rows within one fp16 ulp of the oracle's (a value within a few fp32 ulp
    of an fp16 rounding boundary may land on either side; at most 1% of elements), v cache rows bit-exact, rows
    outside [off, off + T) untouched.
  - bn_gate_rotate (gate_rotate.comp:11-26): within 1e-5 of the oracle (fp32 butterflies in another stage order).
  - the attention layer's four steps chained on the GPU (prep -> attention -> gate_rotate) against the oracle's
    chain: max-abs 2e-3 and the same projected argmax.
"""
import numpy as np
import pytest

import oracle
import workload
from glimpse_language_amd import bonsai_attn as ba

D = 256
pytestmark = pytest.mark.gpu


def inv_freq(theta=1e7, rot=64):
    i = np.arange(rot // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), (2 * i).astype(np.float32) / np.float32(rot))).astype(
        np.float32)


def prep_inputs(seed, T, off, H, KV, mrope=True):
    qp = oracle.normal(seed, 0, (T, H, 512)) * np.float32(2.5)
    kp = oracle.normal(seed, 1, (T, KV, D)) * np.float32(0.7)
    vp = oracle.normal(seed, 2, (T, KV, D))
    qn = (1.0 + 0.1 * oracle.normal(seed, 3, (D,))).astype(np.float32)
    kn = (1.0 + 0.1 * oracle.normal(seed, 4, (D,))).astype(np.float32)
    p = np.arange(off, off + T, dtype=np.int32)
    if mrope:  # image-like rows: h and w positions differ from t
        rng = np.random.default_rng(seed)
        pos = np.stack([p, rng.integers(0, 40000, T), rng.integers(0, 40000, T)]).astype(np.int32)
    else:
        pos = np.stack([p, p, p])
    cap = off + T + 3
    kc = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(seed, 5, (cap, KV, D))))
    vc = oracle.f32_to_f16(oracle.normal(seed, 6, (cap, KV, D)))
    return dict(qp=qp, kp=kp, vp=vp, qn=qn, kn=kn, pos=pos, inv=inv_freq(), kc=kc, vc=vc, off=off)


def to_dev(torch, x):
    if x.dtype == np.uint16:
        x = x.view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def run_prep(torch, ctx, inp, q_dtype=None, in_place=False):
    dev = {k: to_dev(torch, inp[k]) for k in ("qp", "kp", "vp", "qn", "kn", "pos", "inv", "kc", "vc")}
    q = dev["qp"][:, :, :D] if in_place else None
    q = ba.attn_prep(ctx, dev["qp"], dev["kp"], dev["vp"], dev["qn"], dev["kn"], dev["pos"], dev["inv"], dev["kc"],
                     dev["vc"], inp["off"], q=q, q_dtype=q_dtype)
    torch.cuda.synchronize()
    return q, dev


def oracle_prep(inp):
    kc, vc = inp["kc"].copy(), inp["vc"].copy()
    q = oracle.prep(inp["qp"], inp["kp"], inp["vp"], inp["qn"], inp["kn"], inp["pos"], inp["inv"], kc, vc, inp["off"])
    return q, kc, vc


def assert_k_rows_close(got, ref):
    """fp16 bits: equal, or adjacent codes (one ulp apart) in at most 1% of elements."""
    g = got.astype(np.int32)
    r = ref.astype(np.int32)
    diff = np.abs(g - r)
    assert diff.max() <= 1, f"k rows differ by {diff.max()} fp16 ulp"
    assert diff.sum() <= 0.01 * diff.size, f"{diff.sum()} of {diff.size} k elements one ulp off"


@pytest.mark.parametrize("T,off,H,KV,mrope", [
    (1, 1023, 8, 2, False),    # a decode step
    (1, 40000, 16, 4, True),   # late position: large angles
    (5, 3, 8, 2, True),
    (64, 0, 16, 4, True),      # a prefill chunk
    (300, 17, 4, 1, False),
])
def test_prep_matches_oracle(gpu, T, off, H, KV, mrope):
    torch, ctx, _ = gpu
    inp = prep_inputs(0x5E00 + T, T, off, H, KV, mrope)
    print(f"prep T={T} off={off} H={H} KV={KV} mrope={mrope}", flush=True)
    q, dev = run_prep(torch, ctx, inp)
    q_ref, kc_ref, vc_ref = oracle_prep(inp)
    err = float(np.max(np.abs(q.cpu().numpy() - q_ref)))
    assert err <= 3e-5, err
    kc = dev["kc"].cpu().numpy().view(np.uint16)
    vc = dev["vc"].cpu().numpy().view(np.uint16)
    rows = slice(off, off + T)
    assert_k_rows_close(kc[rows], kc_ref[rows])
    assert np.array_equal(vc[rows], vc_ref[rows])
    # rows outside [off, off + T) keep their contents
    assert np.array_equal(kc[:off], inp["kc"][:off]) and np.array_equal(kc[off + T:], inp["kc"][off + T:])
    assert np.array_equal(vc[:off], inp["vc"][:off]) and np.array_equal(vc[off + T:], inp["vc"][off + T:])


@pytest.mark.parametrize("T,off,H,KV,rot,s1,s2", [
    (3, 50, 32, 8, 256, 24, 20),    # 48 head rows per token: two blocks each; 128 pair angles (two per lane)
    (70, 5, 32, 8, 200, 30, 30),    # long-prompt grid, each wave over three rounds of rows; 100 pair angles
    (9, 0, 4, 1, 128, 11, 11),      # exactly 64 pair angles
    (1, 123, 64, 16, 64, 11, 11),   # 96 head rows: four blocks for the one token
    (2, 9, 8, 2, 0, 0, 0),          # no rotation
])
def test_prep_rotation_widths_and_head_counts(gpu, T, off, H, KV, rot, s1, s2):
    torch, ctx, _ = gpu
    inp = prep_inputs(0x5E40 + T + H, T, off, H, KV, mrope=True)
    inp["inv"] = inv_freq(rot=max(rot, 8))
    print(f"prep T={T} off={off} H={H} KV={KV} rot={rot} s1={s1} s2={s2}", flush=True)
    dev = {k: to_dev(torch, inp[k]) for k in ("qp", "kp", "vp", "qn", "kn", "pos", "inv", "kc", "vc")}
    q = ba.attn_prep(ctx, dev["qp"], dev["kp"], dev["vp"], dev["qn"], dev["kn"], dev["pos"], dev["inv"], dev["kc"],
                     dev["vc"], off, rot, s1, s2)
    torch.cuda.synchronize()
    kc_ref, vc_ref = inp["kc"].copy(), inp["vc"].copy()
    q_ref = oracle.prep(inp["qp"], inp["kp"], inp["vp"], inp["qn"], inp["kn"], inp["pos"], inp["inv"], kc_ref, vc_ref,
                        off, rot, s1, s2)
    err = float(np.max(np.abs(q.cpu().numpy() - q_ref)))
    assert err <= 3e-5, err
    kc = dev["kc"].cpu().numpy().view(np.uint16)
    vc = dev["vc"].cpu().numpy().view(np.uint16)
    rows = slice(off, off + T)
    assert_k_rows_close(kc[rows], kc_ref[rows])
    assert np.array_equal(vc[rows], vc_ref[rows])
    assert np.array_equal(kc[:off], inp["kc"][:off]) and np.array_equal(kc[off + T:], inp["kc"][off + T:])


def test_prep_fp16_q_and_in_place(gpu):
    torch, ctx, _ = gpu
    inp = prep_inputs(0x5E77, 9, 100, 8, 2)
    q32, _ = run_prep(torch, ctx, inp)
    q16, _ = run_prep(torch, ctx, inp, q_dtype=torch.float16)
    assert q16.dtype == torch.float16
    assert torch.equal(q16, q32.half())
    qp_before = to_dev(torch, inp["qp"])
    q_in, dev = run_prep(torch, ctx, inp, in_place=True)
    assert torch.equal(q_in, q32)                                  # q written over the q half of qp
    assert torch.equal(dev["qp"][:, :, D:], qp_before[:, :, D:])   # the gate half untouched


def test_prep_rejects_bad_args(gpu):
    torch, ctx, _ = gpu
    inp = prep_inputs(0x5E78, 2, 0, 4, 1)
    dev = {k: to_dev(torch, inp[k]) for k in ("qp", "kp", "vp", "qn", "kn", "pos", "inv", "kc", "vc")}
    q = torch.empty((2, 4, D), dtype=torch.float32, device="cuda")
    a = ba.prep_args(dev["qp"], dev["kp"], dev["vp"], dev["qn"], dev["kn"], dev["pos"], dev["inv"], q, dev["kc"],
                     dev["vc"], 0, rot=60)
    with pytest.raises(ba.BonsaiAttnError):
        ctx.call("bn_attn_prep", a)
    assert "rot" in ctx.error()


def rotate_inputs(seed, T, H):
    W = H * D
    attn = oracle.normal(seed, 0, (T, W))
    qp = oracle.normal(seed, 1, (T, H, 512)) * np.float32(2.0)
    signs = np.where(oracle.normal(seed, 2, (W,)) > 0, 1.0, -1.0).astype(np.float32)
    return attn, qp, signs


@pytest.mark.parametrize("T,H", [(1, 16), (7, 8), (33, 2), (4096, 16)])
def test_gate_rotate_matches_oracle(gpu, T, H):
    torch, ctx, _ = gpu
    attn, qp, signs = rotate_inputs(0x6A00 + T, T, H)
    print(f"gate_rotate T={T} H={H}", flush=True)
    d_attn, d_qp, d_signs = to_dev(torch, attn), to_dev(torch, qp), to_dev(torch, signs)
    xr = ba.gate_rotate(ctx, d_attn, d_signs, gate=d_qp[:, :, D:])
    torch.cuda.synchronize()
    rows = np.arange(T) if T <= 64 else np.r_[0:8, T - 8:T]
    ref = oracle.gate_rotate(attn[rows], qp[rows].reshape(len(rows), -1), signs)
    err = float(np.max(np.abs(xr.cpu().numpy()[rows] - ref)))
    assert err <= 1e-5, err
    if T > 64:  # every row: the transform is orthogonal, so it keeps the gated row's norm
        g = torch.sigmoid(d_qp[:, :, D:].reshape(T, -1)) * d_attn
        n_in = torch.linalg.vector_norm(g.double(), dim=1)
        n_out = torch.linalg.vector_norm(xr.double(), dim=1)
        assert float(torch.max(torch.abs(n_out / n_in - 1))) < 1e-5


def test_gate_rotate_pre_gated_and_in_place(gpu):
    torch, ctx, _ = gpu
    attn, qp, signs = rotate_inputs(0x6A99, 5, 8)
    d_attn, d_qp, d_signs = to_dev(torch, attn), to_dev(torch, qp), to_dev(torch, signs)
    ref = ba.gate_rotate(ctx, d_attn, d_signs, gate=d_qp[:, :, D:])
    gated = d_attn * torch.sigmoid(d_qp[:, :, D:].reshape(5, -1))
    pre = ba.gate_rotate(ctx, gated, d_signs)                         # gate == NULL: attn already gated
    ba.gate_rotate(ctx, d_attn, d_signs, gate=d_qp[:, :, D:], xr=d_attn)  # xr over attn
    torch.cuda.synchronize()
    assert float(torch.max(torch.abs(pre - ref))) <= 1e-5
    assert torch.equal(d_attn, ref)


@pytest.mark.parametrize("T,off", [(1, 2047), (8, 1000), (200, 300)])
def test_layer_chain_matches_oracle(gpu, T, off):
    """attn_prep -> attention -> gate_rotate on the GPU vs the oracle's chain (model.rs:815-894)."""
    torch, ctx, ws = gpu
    H, KV = 8, 2
    W = H * D
    inp = prep_inputs(0x7C00 + T, T, off, H, KV)
    signs = np.where(oracle.normal(0x7C00 + T, 9, (W,)) > 0, 1.0, -1.0).astype(np.float32)
    print(f"layer chain T={T} off={off}", flush=True)
    q, dev = run_prep(torch, ctx, inp)
    attn = ba.attention(ctx, ws, q, dev["kc"], dev["vc"], off)
    xr = ba.gate_rotate(ctx, attn.reshape(T, W), to_dev(torch, signs), gate=dev["qp"][:, :, D:])
    torch.cuda.synchronize()
    q_ref, kc_ref, vc_ref = oracle_prep(inp)
    attn_ref = oracle.attend(q_ref, kc_ref, vc_ref, off)
    ref = oracle.gate_rotate(attn_ref.reshape(T, W), inp["qp"].reshape(T, -1), signs)
    attn16 = oracle.attend(q_ref, kc_ref, vc_ref, off, p16=True)
    ref16 = oracle.gate_rotate(attn16.reshape(T, W), inp["qp"].reshape(T, -1), signs)
    out = xr.cpu().numpy()
    err = float(np.max(np.abs(out - ref)))
    assert err <= 2e-3, err
    R = oracle.normal(workload.PROJ_SEED, 0, (W, 128)).astype(np.float64)
    bad, ties = workload.argmax_mismatches(out, ref, R, ref16)
    assert len(bad) == 0, f"projected argmax differs on rows {bad}"
