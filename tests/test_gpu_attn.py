"""Parity of the HIP attention path (through the C ABI) with the oracle, on the GPU.

Bar (from the task): outputs within max-abs 2e-3 of the oracle (fp32 accumulate), an identical argmax of
each output row projected by a fixed random matrix (rows whose two best projected reference values lie within
3 sqrt(2) |ref16 - ref| are ties, not compared, at most max(2, rows / 100) of them; ref16 is the oracle with
fp16-rounded probabilities, so the margin does not depend on the output under test), bit-exact fp16 cache rows
after the append, and bit-identical results across repeated runs.
"""
import numpy as np
import pytest

import oracle
import workload
from glimpse_language_amd import bonsai_attn as ba

pytestmark = pytest.mark.gpu

TOL = 2e-3  # max-abs tolerance against the oracle


def to_dev(torch, inp):
    d = {}
    for k in ("q", "k_new", "v_new", "gate"):
        d[k] = None if inp[k] is None else torch.from_numpy(np.ascontiguousarray(inp[k])).cuda()
    d["kc"] = torch.from_numpy(inp["kc"].view(np.int16).copy()).cuda()
    d["vc"] = torch.from_numpy(inp["vc"].view(np.int16).copy()).cuda()
    return d


def run(gpu, inp, kind=ba.KIND_FORWARD, append=True, dev=None):
    torch, ctx, ws = gpu
    d = dev or to_dev(torch, inp)
    out = ba.attention(ctx, ws, d["q"], d["kc"], d["vc"], inp["off"], k_new=d["k_new"] if append else None,
                       v_new=d["v_new"] if append else None, gate=d["gate"], kind=kind)
    torch.cuda.synchronize()
    return out.cpu().numpy(), d


def cache_np(t):
    return t.cpu().numpy().view(np.uint16)


def assert_parity(out, ref, H, what, ref16):
    """max-abs within TOL and the projected argmax equal on every row that is not a tie; ties are sized by the
    perturbed oracle ref16 (probabilities rounded to fp16), not by `out`, and printed."""
    err = float(np.max(np.abs(out - ref)))
    assert err <= TOL, f"{what} max-abs {err:.3e} > {TOL}"
    R = workload.projection(H)
    bad, ties = workload.argmax_mismatches(out, ref, R, ref16)
    rows = ref.shape[0]
    print(f"{what}: max-abs {err:.3e}; argmax on {rows} rows, {len(ties)} tie rows excused {ties.tolist()[:32]}",
          flush=True)
    assert len(bad) == 0, f"{what} projected argmax differs in rows {bad[:8]}"
    assert len(ties) <= workload.tie_cap(rows), f"{what}: {len(ties)} tie rows"
    return err


def check_case(gpu, inp, kind=ba.KIND_FORWARD, rows=None):
    out, d = run(gpu, inp, kind)
    ref, kc_ref, vc_ref = workload.expected(inp, rows=rows)
    ref16, _, _ = workload.expected(inp, rows=rows, p16=True)
    T = inp["T"]
    got = out if rows is None else out[list(rows)]
    err = assert_parity(got, ref, inp["H"], f"T={T} off={inp['off']}", ref16)
    assert np.array_equal(cache_np(d["kc"]), kc_ref), "K cache differs after the append"
    assert np.array_equal(cache_np(d["vc"]), vc_ref), "V cache differs after the append"
    # repeat on the updated cache without the append: same bits
    out2, _ = run(gpu, inp, kind, append=False, dev=d)
    assert np.array_equal(out, out2), "repeat run not bit-identical"
    return err


@pytest.mark.parametrize("L", [1, 2, 15, 16, 17, 63, 64, 65, 100, 1000, 1024, 4097, 9000])
def test_decode_lengths(gpu, L):
    inp = workload.layer(workload.SEED_BASE + L, T=1, off=L - 1, H=8, KV=2)
    check_case(gpu, inp, ba.KIND_DECODE)


def test_decode_1k_workload(gpu):
    inp = workload.layer(workload.SEED_BASE + 0, **{k: v for k, v in workload.WORKLOADS["decode_1k"].items()})
    err = check_case(gpu, inp, ba.KIND_DECODE)
    print(f"decode_1k max-abs {err:.3e}")


def test_decode_4b_heads_no_gate(gpu):
    inp = workload.layer(77, T=1, off=3000, H=16, KV=4, gate=False)
    check_case(gpu, inp, ba.KIND_DECODE)


def test_decode_without_append_reads_cache_row(gpu):
    inp = workload.layer(78, T=1, off=500, H=8, KV=2)
    kc, vc = inp["kc"].copy(), inp["vc"].copy()
    oracle.append(inp["k_new"], inp["v_new"], kc, vc, inp["off"])
    inp2 = dict(inp, kc=kc, vc=vc)
    out, _ = run(gpu, inp2, ba.KIND_DECODE, append=False)
    ref = oracle.attend(inp["q"], kc, vc, inp["off"], inp["gate"])
    assert_parity(out, ref, 8, "decode from the cache", oracle.attend(inp["q"], kc, vc, inp["off"], inp["gate"], p16=True))


def test_gate_in_place_from_qproj(gpu):
    torch, ctx, ws = gpu
    inp = workload.layer(79, T=1, off=700, H=8, KV=2)
    qp = oracle.normal(79, 9, (1, 8, 512))
    d = to_dev(torch, inp)
    qp_d = torch.from_numpy(qp).cuda()
    out = ba.attention(ctx, ws, d["q"], d["kc"], d["vc"], inp["off"], k_new=d["k_new"], v_new=d["v_new"],
                       gate=qp_d[:, :, 256:], g_strides=(8 * 512, 512))
    torch.cuda.synchronize()
    ref, _, _ = workload.expected(dict(inp, gate=qp[:, :, 256:]))
    ref16, _, _ = workload.expected(dict(inp, gate=qp[:, :, 256:]), p16=True)
    assert_parity(out.cpu().numpy(), ref, 8, "gate from the q projection", ref16)


def test_verify_8_workload(gpu):
    inp = workload.layer(workload.SEED_BASE + 2, **workload.WORKLOADS["verify_8"])
    check_case(gpu, inp, ba.KIND_VERIFY)


# (2, 0), (3, 17): short contexts, rows as decodes of one split; the rest run on verify_kernel: one split (2, 63), a
# partial last tile (6, 129), many splits; 9..16 rows as two row groups (the second one partial for 9 and 12 rows)
@pytest.mark.parametrize("T,off", [(2, 0), (3, 17), (16, 1000), (5, 4095), (2, 63), (6, 129), (7, 1000), (8, 9000),
                                   (9, 500), (12, 3000), (16, 70), (15, 9000)])
def test_verify_shapes(gpu, T, off):
    inp = workload.layer(900 + T + off, T=T, off=off, H=8, KV=2)
    check_case(gpu, inp, ba.KIND_VERIFY)


@pytest.mark.parametrize("T,off,gate", [(8, 8191, True), (3, 2000, False), (4, 250, True), (16, 8176, True)])
def test_verify_4b_heads(gpu, T, off, gate):
    inp = workload.layer(950 + T + off, T=T, off=off, H=16, KV=4, gate=gate)
    check_case(gpu, inp, ba.KIND_VERIFY)


def test_verify_rows_equal_decodes(gpu):
    """Row t of a verify call matches a decode at off+t: the equivalence the runtime's accept relies on.

    The verify kernel multiplies fp16 q and p on the MFMA units while the decode kernel carries q as an fp16
    hi/lo pair (fp32-accurate scores), so the two agree to a few 1e-5 (each is within 2e-3 of the oracle);
    2e-4 bounds their difference."""
    inp = workload.layer(31, T=6, off=800, H=8, KV=2)
    out, d = run(gpu, inp, ba.KIND_VERIFY)
    torch, ctx, ws = gpu
    for t in range(6):
        o = ba.attention(ctx, ws, d["q"][t:t + 1], d["kc"], d["vc"], inp["off"] + t,
                         gate=d["gate"][t:t + 1], kind=ba.KIND_DECODE)
        torch.cuda.synchronize()
        assert np.max(np.abs(o.cpu().numpy()[0] - out[t])) <= 2e-4


@pytest.mark.parametrize("T", [8, 16])
def test_verify_kernel_equals_rows_path(gpu, T):
    """verify_kernel (8 rows of a kv head in one MFMA tile, each K/V row read once per 8 rows) against the same call
    run as decodes of its rows (BONSAI_ATTN_VERIFY_MFMA=0): both carry the reference's semantics, and differ only by
    the fp16 rounding of q in the MFMA scores (a few 1e-5); 2e-4 bounds it."""
    from conftest import context_with
    torch, ctx, ws = gpu
    inp = workload.layer(0x9500 + T, T=T, off=8192 - T, H=16, KV=4)
    out, d = run(gpu, inp, ba.KIND_VERIFY)
    ctx0 = context_with(BONSAI_ATTN_VERIFY_MFMA=0)
    ws0 = ba.Workspace(ctx0, "cuda")
    rows = ba.attention(ctx0, ws0, d["q"], d["kc"], d["vc"], inp["off"], gate=d["gate"], kind=ba.KIND_VERIFY)
    torch.cuda.synchronize()
    assert np.max(np.abs(rows.cpu().numpy() - out)) <= 2e-4


@pytest.mark.parametrize("T,off,H,KV", [(40, 3000, 16, 4), (64, 100, 8, 2), (17, 0, 4, 1)])
def test_mid_rows_equal_flash(gpu, T, off, H, KV):
    """17..64 rows take verify_kernel's row groups of 8 (BONSAI_ATTN_MID_ROWS, on by default) instead of
    flash_kernel: both against the oracle, and against each other within 2e-4 (both carry an fp32 q as an fp16 hi/lo
    pair; they differ in the order of the sums)."""
    from conftest import context_with
    torch, ctx, ws = gpu
    inp = workload.layer(0x9700 + T + off, T=T, off=off, H=H, KV=KV)
    print(f"mid rows vs flash: T={T} off={off} H={H} KV={KV}", flush=True)
    err = check_case(gpu, inp, ba.KIND_PREFILL)
    out, d = run(gpu, inp, ba.KIND_PREFILL, append=False)
    ctx0 = context_with(BONSAI_ATTN_MID_ROWS=0)
    ws0 = ba.Workspace(ctx0, "cuda")
    fl = ba.attention(ctx0, ws0, d["q"], d["kc"], d["vc"], inp["off"], gate=d["gate"], kind=ba.KIND_PREFILL)
    torch.cuda.synchronize()
    diff = float(np.max(np.abs(fl.cpu().numpy() - out)))
    print(f"mid rows vs flash: oracle max-abs {err:.3e}, paths differ by {diff:.3e}", flush=True)
    assert diff <= 2e-4
    ctx0.close()


def test_prefill_prefix_workload(gpu):
    inp = workload.layer(workload.SEED_BASE + 1, **workload.WORKLOADS["prefill_prefix"])
    err = check_case(gpu, inp, ba.KIND_PREFILL)
    print(f"prefill_prefix max-abs {err:.3e}")


@pytest.mark.parametrize("T,off,H,KV", [(17, 0, 4, 1), (33, 5, 8, 2), (100, 300, 16, 4)])
def test_prefill_shapes(gpu, T, off, H, KV):
    inp = workload.layer(1000 + T + off, T=T, off=off, H=H, KV=KV)
    check_case(gpu, inp, ba.KIND_PREFILL)


def test_prefill_4k_workload_sampled_rows(gpu):
    """Full 4096-row prefill on the GPU; the oracle checks a spread of rows (decode-equivalent rows)."""
    inp = workload.layer(workload.SEED_BASE + 3, **workload.WORKLOADS["prefill_4k"])
    rows = sorted(set([0, 1, 2, 63, 64, 127, 128, 1000, 2047, 2048, 3001, 4094, 4095] +
                      list(np.random.default_rng(5).integers(0, 4096, 20))))
    err = check_case(gpu, inp, ba.KIND_PREFILL, rows=rows)
    print(f"prefill_4k sampled rows max-abs {err:.3e}")


def make_ragged(seed, nseq, H, KV, lo, hi):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=nseq).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    rows = int(lens.sum())
    kc = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(seed, 2, (rows, KV, 256))))
    vc = oracle.f32_to_f16(oracle.normal(seed, 3, (rows, KV, 256)))
    q = oracle.rms_rows(oracle.normal(seed, 1, (nseq, H, 256)))
    k_new = oracle.rms_rows(oracle.normal(seed, 4, (nseq, KV, 256)))
    v_new = oracle.normal(seed, 5, (nseq, KV, 256))
    z = oracle.normal(seed, 6, (nseq, H, 256))
    return lens, offs, kc, vc, q, k_new, v_new, z


@pytest.mark.parametrize("nseq,lo,hi", [(1, 1, 1), (7, 1, 300), (32, 1024, 4096), (5, 4000, 20000),
                                        (100, 1, 400), (130, 60, 70)])
def test_ragged_decode(gpu, nseq, lo, hi):
    run_ragged(gpu, *make_ragged(nseq * 1000 + hi, nseq, 16, 4, lo, hi))


def test_ragged_decode_one_long_many_short(gpu):
    """Balanced splits on a lopsided batch: one 30000-key sequence among 70 short ones (the long one takes
    most of the splits; more than 64 sequences take the multi-pass scan of the lengths)."""
    nseq, H, KV = 71, 8, 2
    lens, offs, kc, vc, q, k_new, v_new, z = make_ragged(4711, nseq, H, KV, 1, 90)
    lens[37] = 30000
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    rows = int(lens.sum())
    kc = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(4711, 2, (rows, KV, 256))))
    vc = oracle.f32_to_f16(oracle.normal(4711, 3, (rows, KV, 256)))
    run_ragged(gpu, lens, offs, kc, vc, q, k_new, v_new, z)


def run_ragged(gpu, lens, offs, kc, vc, q, k_new, v_new, z):
    torch, ctx, ws = gpu
    nseq, H = q.shape[0], q.shape[1]
    kc_ref, vc_ref = kc.copy(), vc.copy()
    for i in range(nseq):  # the new row of sequence i goes to its last row
        r = offs[i] + lens[i] - 1
        kc_ref[r] = k_new[i].astype(np.float16).view(np.uint16)
        vc_ref[r] = v_new[i].astype(np.float16).view(np.uint16)
    ref = oracle.decode_ragged(q, kc_ref, vc_ref, offs, lens, z)
    ref16 = oracle.decode_ragged(q, kc_ref, vc_ref, offs, lens, z, p16=True)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    kc_d, vc_d = t(kc.view(np.int16)), t(vc.view(np.int16))
    out = ba.decode_ragged(ctx, ws, t(q), kc_d, vc_d, t(offs), t(lens), int(lens.max()), k_new=t(k_new),
                           v_new=t(v_new), gate=t(z))
    torch.cuda.synchronize()
    assert_parity(out.cpu().numpy(), ref, H, "ragged", ref16)
    assert np.array_equal(cache_np(kc_d), kc_ref)
    assert np.array_equal(cache_np(vc_d), vc_ref)


def test_workspace_reused_across_shapes(gpu):
    """One workspace serves calls of different shapes in turn: the split counters stay at zero between calls
    and no call's partial records overlap them."""
    torch, ctx, _ = gpu
    ws = ba.Workspace(ctx, "cuda")
    ws.get(64 << 20)  # large enough for every call below, so the same bytes are reused
    for seed, (T, off, H, KV) in enumerate([(100, 700, 8, 2), (1, 8999, 8, 2), (1, 3000, 16, 4), (7, 4000, 16, 4)]):
        inp = workload.layer(4242 + seed, T=T, off=off, H=H, KV=KV)
        d = to_dev(torch, inp)
        out = ba.attention(ctx, ws, d["q"], d["kc"], d["vc"], off, k_new=d["k_new"], v_new=d["v_new"],
                           gate=d["gate"])
        torch.cuda.synchronize()
        ref, _, _ = workload.expected(inp)
        ref16, _, _ = workload.expected(inp, p16=True)
        assert_parity(out.cpu().numpy(), ref, H, f"reuse T={T} off={off}", ref16)
    lens, offs, kc, vc, q, k_new, v_new, z = make_ragged(99, 32, 16, 4, 1024, 4096)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = ba.decode_ragged(ctx, ws, t(q), t(kc.view(np.int16)), t(vc.view(np.int16)), t(offs), t(lens),
                           int(lens.max()))
    torch.cuda.synchronize()
    assert_parity(out.cpu().numpy(), oracle.decode_ragged(q, kc, vc, offs, lens), 16, "reuse ragged",
                  oracle.decode_ragged(q, kc, vc, offs, lens, p16=True))


def test_bad_arguments_do_not_launch(gpu):
    torch, ctx, ws = gpu
    inp = workload.layer(5, T=2, off=10, H=8, KV=2)
    d = to_dev(torch, inp)
    with pytest.raises(ba.BonsaiAttnError) as e:
        ba.attention(ctx, ws, d["q"], d["kc"], d["vc"], 10, kind=ba.KIND_DECODE)  # T=2 is not a decode
    assert e.value.status == ba.BN_EINVAL
    a = ba.attn_args(1, 5000, 8, 2, 5001, d["q"], d["kc"], d["vc"], d["q"])
    with pytest.raises(ba.BonsaiAttnError) as e:
        ctx.call("bn_attn_decode", a)  # needs a workspace
    assert e.value.status == ba.BN_ENOWS
