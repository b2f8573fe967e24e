"""bn_ternary_matmul (the q/k/v/o projections, model.rs:455-596) against the oracle's qmm3-order fp32 matmul.

Every output is within workload.ternary_tolerance of the oracle: 2e-5 of the L2 norm of its K products (fp32 sums in
another order differ by about 3e-6 of it; a path that rounded x to fp16 would be off by about 2.4e-4), and within the
north-star max-abs 2e-3. Repeated calls are bit-identical. Cases cover each kernel: the VALU rows kernel (T = 1..4),
the split-K MFMA kernel (T = 5..32, K split 8, 4 or 2 ways), the 128-token MFMA kernel (T > 32, partly empty token
and row tiles), and for T > 32 with a workspace the split-once pair (tern_split_kernel + tern_pf_kernel), whose
results must equal the in-place kernel's bit for bit; one to three matrices sharing x, add into y, LoRA, code 3 and
strided rows.
"""
import numpy as np
import pytest

import oracle
import workload
from glimpse_language_amd import bonsai_attn as ba

pytestmark = pytest.mark.gpu


def make_case(seed, T, K, os, code3=False, lora_r=0, x_pad=0):
    mats = [workload.ternary_weights(seed + 17 * i, o, K, code3) for i, o in enumerate(os)]
    x = oracle.normal(seed, 1, (T, K + x_pad))
    lb = [oracle.f32_to_f16(oracle.normal(seed + i, 2, (o, lora_r))) for i, o in enumerate(os)] if lora_r else None
    lu = oracle.normal(seed, 3, (T, len(os) * lora_r)) if lora_r else None
    return mats, x, lb, lu


def run_gpu(torch, ctx, mats, x, K, add_y=None, lb=None, lu=None, lora_r=0, work=False):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    xd = dev(x)[:, :K]
    ys, margs = [], []
    for i, (w, s, _) in enumerate(mats):
        y = dev(add_y[i]) if add_y is not None else torch.full((x.shape[0], w.shape[0]), float("nan"), device="cuda")
        ys.append(y)
        m = [dev(w.view(np.int32)), dev(s.view(np.int16)), y]
        if lb is not None:
            m.append(dev(lb[i].view(np.int16)))
        margs.append(tuple(m))
    ws = ba.ternary_workspace(xd) if work else None
    if work:
        assert ws is not None and x.shape[0] > 32
        ws.fill_(0xA5)  # stale contents must not matter
    ba.ternary_matmul(ctx, xd, margs, add=add_y is not None, lora_u=None if lu is None else dev(lu), lora_r=lora_r,
                      work=ws)
    torch.cuda.synchronize()
    return [y.cpu().numpy() for y in ys]


def expected(mats, x, K, add_y=None, lb=None, lu=None, lora_r=0):
    out = []
    for i, (w, s, _) in enumerate(mats):
        u = None if lu is None else lu[:, i * lora_r:(i + 1) * lora_r]
        out.append(oracle.ternary(w, s, x[:, :K], y=None if add_y is None else add_y[i],
                                  lora_b=None if lb is None else lb[i], lora_u=u))
    return out


def check(got, ref, mats, x, K, what, abs_bar=True, cancel=False):
    for i, (g, r) in enumerate(zip(got, ref)):
        w, s, codes = mats[i]
        tol = workload.ternary_tolerance(x[:, :K], codes, s)
        if cancel:
            # the rows kernel's s (sum x c - sum x) (qmv.glsl:22-35) cancels the sum of x where codes are 1: its
            # fp32 rounding scales with s sum |x|, not with the products
            smax = oracle.f16_to_f32(s).astype(np.float64).max(axis=1)
            tol = tol + 2.0 ** -20 * np.abs(x[:, :K]).astype(np.float64).sum(axis=1)[:, None] * smax[None, :]
        err = np.abs(g.astype(np.float64) - r)
        bad = np.argwhere(~(err <= tol))
        assert bad.size == 0, f"{what} mat {i}: {len(bad)} outputs off, first {bad[:3].tolist()}, max err {err.max()}"
        if abs_bar:
            assert err.max() <= 2e-3


# (T, K, output rows per matrix)
CASES = [
    (1, 2048, (4096, 512, 512)),   # 2B q/k/v decode step
    (1, 2560, (2560,)),            # 4B o_proj-sized decode
    (2, 2048, (512,)), (3, 384, (64, 128)), (4, 1024, (192,)),
    (5, 2048, (256,)), (8, 2560, (8192, 1024, 1024)),   # 4B verify rows: K split 8 ways (fewer tiles than CUs)
    (6, 768, (128,)),              # K split 4 ways (768 = 4 * 192)
    (16, 384, (64, 64, 64)),       # K split 2 ways (384 = 2 * 192)
    (12, 640, (128,)),             # K split 2 ways (640 = 2 * 320, scale groups straddle the halves)
    (32, 2048, (512,)), (33, 256, (704,)),              # first 128-token tile: partly empty token and row tiles
    (130, 2048, (512, 128, 128)), (300, 1024, (320,)),
    (1, 128, (64,)), (8, 128, (64,)), (40, 128, (128,)),   # K = 128: one scale group, one or two chunks
]


@pytest.mark.parametrize("T,K,os", CASES)
def test_ternary_matches_oracle(gpu, T, K, os):
    torch, ctx, _ = gpu
    print(f"ternary T={T} K={K} os={os}", flush=True)
    mats, x, _, _ = make_case(0x7000 + T + K, T, K, os)
    got = run_gpu(torch, ctx, mats, x, K)
    check(got, expected(mats, x, K), mats, x, K, f"T={T} K={K}")
    again = run_gpu(torch, ctx, mats, x, K)
    assert all(np.array_equal(a, b) for a, b in zip(got, again)), "repeat call not bit-identical"


# T > 32 shapes for the split-once pair: a partial last token tile, K = 128 (two chunks, one scale group), K = 640
# (ten chunks, odd scale-group count per row), a second row member straddling a 256-row block, the 4B q/k/v shape
SPLIT_CASES = [(33, 256, (704,)), (40, 128, (128,)), (100, 640, (192, 64)), (130, 2048, (512, 128, 128)),
               (300, 1024, (320,)), (257, 2560, (8192, 1024, 1024))]


@pytest.mark.parametrize("T,K,os", SPLIT_CASES)
def test_ternary_split_once_matches_in_place(gpu, T, K, os):
    torch, ctx, _ = gpu
    print(f"ternary split-once T={T} K={K} os={os}", flush=True)
    mats, x, _, _ = make_case(0x7400 + T + K, T, K, os)
    got = run_gpu(torch, ctx, mats, x, K, work=True)
    check(got, expected(mats, x, K), mats, x, K, f"split-once T={T} K={K}")
    ref = run_gpu(torch, ctx, mats, x, K)
    assert all(np.array_equal(a, b) for a, b in zip(got, ref)), "split-once and in-place results differ"
    again = run_gpu(torch, ctx, mats, x, K, work=True)
    assert all(np.array_equal(a, b) for a, b in zip(got, again)), "repeat call not bit-identical"


def test_ternary_split_once_large_grid(gpu):
    """A split-once call whose grid of 64-token blocks exceeds three per CU (1,300 tokens x 10,240 rows: 840 blocks)
    takes the 128-token blocks of tern_pf_kernel (two x tiles per block; 21 x tiles, so the last block has one and a
    short one), the smaller shapes above the 64-token blocks: bit-identical to the in-place kernel, and the first 64
    rows of each matrix checked against the oracle. Then the same with a few x values beyond fp16's range, in a token
    of each x tile of one block and in the last token (the scaled pass over both of a block's x tiles)."""
    torch, ctx, _ = gpu
    T, K, os = 1300, 2560, (8192, 1024, 1024)
    print(f"ternary split-once large grid T={T}", flush=True)
    mats, x, _, _ = make_case(0x7700, T, K, os)
    got = run_gpu(torch, ctx, mats, x, K, work=True)
    ref = run_gpu(torch, ctx, mats, x, K)
    assert all(np.array_equal(a, b) for a, b in zip(got, ref)), "split-once and in-place results differ"
    head = [(w[:64], sc[:64], codes[:64]) for w, sc, codes in mats]
    check([g[:, :64] for g in got], expected(head, x, K), head, x, K, "large grid, first rows")
    print(f"ternary split-once large grid T={T}, x beyond fp16", flush=True)
    x = x.copy()
    x[130, 7], x[200, 1500], x[T - 1, K - 1] = 1.0e5, -7.0e6, 4.0e4
    got = run_gpu(torch, ctx, mats, x, K, work=True)
    ref = run_gpu(torch, ctx, mats, x, K)
    assert all(np.array_equal(a, b) for a, b in zip(got, ref)), "split-once and in-place results differ (large x)"


def test_ternary_workspace_with_unaligned_scales(gpu):
    """A scale array that is only 2-byte aligned cannot be copied 4 bytes at a time: with a workspace the call then
    takes the in-place kernel, with the same results."""
    torch, ctx, _ = gpu
    T, K, os = 70, 512, (128,)
    mats, x, _, _ = make_case(0x7600, T, K, os)
    w, sc, _ = mats[0]
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    wd = torch.from_numpy(np.ascontiguousarray(w.view(np.int32))).cuda()
    flat = torch.zeros(sc.size + 1, dtype=torch.int16, device="cuda")
    flat[1:] = torch.from_numpy(np.ascontiguousarray(sc.view(np.int16)).reshape(-1)).cuda()
    sd = flat[1:].view(sc.shape)
    assert sd.data_ptr() % 4 == 2
    ys = []
    for work in (None, ba.ternary_workspace(xd)):
        y = torch.full((T, os[0]), float("nan"), device="cuda")
        ba.ternary_matmul(ctx, xd, [(wd, sd, y)], work=work)
        ys.append(y)
    torch.cuda.synchronize()
    got = [y.cpu().numpy() for y in ys]
    assert np.array_equal(got[0], got[1])
    check([got[1]], expected(mats, x, K), mats, x, K, "unaligned scales")


def test_ternary_workspace_size_and_check(gpu):
    torch, ctx, _ = gpu
    assert ba.ternary_workspace_size(32, 2048) == 0 and ba.ternary_workspace_size(1, 2048) == 0
    assert ba.ternary_workspace_size(33, 256) == 1 * 4 * (16384 + 4)
    assert ba.ternary_workspace_size(4096, 2560) == 64 * 40 * (16384 + 4)
    mats, x, _, _ = make_case(0x7500, 64, 256, (64,))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    xd, y = dev(x), torch.zeros((64, 64), device="cuda")
    m = [(dev(mats[0][0].view(np.int32)), dev(mats[0][1].view(np.int16)), y)]
    ws = ba.ternary_workspace(xd)
    small = ba.ternary_args(xd, m, work=ws[:-4])
    assert ba.load().bn_ternary_check(small) == ba.BN_EINVAL
    unaligned = ba.ternary_args(xd, m, work=ws[16:])
    assert ba.load().bn_ternary_check(unaligned) == ba.BN_EINVAL
    assert ba.load().bn_ternary_check(ba.ternary_args(xd, m, work=ws)) == ba.BN_OK


@pytest.mark.parametrize("T", [1, 3, 8, 40])
def test_ternary_add_lora_code3_strided(gpu, T):
    torch, ctx, _ = gpu
    K, os, r = 512, (128, 64), 6
    print(f"ternary add/lora T={T}", flush=True)
    mats, x, lb, lu = make_case(0x7100 + T, T, K, os, code3=True, lora_r=r, x_pad=12)
    y0 = [oracle.normal(0x7100 + T, 5 + i, (T, o)) for i, o in enumerate(os)]
    got = run_gpu(torch, ctx, mats, x, K, add_y=y0, lb=lb, lu=lu, lora_r=r)
    check(got, expected(mats, x, K, add_y=y0, lb=lb, lu=lu, lora_r=r), mats, x, K, f"add/lora T={T}")
    if T > 32:
        once = run_gpu(torch, ctx, mats, x, K, add_y=y0, lb=lb, lu=lu, lora_r=r, work=True)
        assert all(np.array_equal(a, b) for a, b in zip(got, once)), "split-once and in-place results differ"


def test_ternary_one_matrix_without_lora(gpu):
    """With a LoRA rank set, a matrix with lora_b = NULL gets no up projection (the reference's zero B)."""
    torch, ctx, _ = gpu
    T, K, os, r = 2, 256, (64, 64), 4
    mats, x, lb, lu = make_case(0x7200, T, K, os, lora_r=r)
    lb_none = [lb[0], None]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    ys = [torch.zeros((T, o), device="cuda") for o in os]
    margs = [(dev(mats[0][0].view(np.int32)), dev(mats[0][1].view(np.int16)), ys[0], dev(lb[0].view(np.int16))),
             (dev(mats[1][0].view(np.int32)), dev(mats[1][1].view(np.int16)), ys[1])]
    ba.ternary_matmul(ctx, dev(x), margs, lora_u=dev(lu), lora_r=r)
    torch.cuda.synchronize()
    ref = [oracle.ternary(mats[0][0], mats[0][1], x, lora_b=lb_none[0], lora_u=lu[:, :r]),
           oracle.ternary(mats[1][0], mats[1][1], x)]
    check([y.cpu().numpy() for y in ys], ref, mats, x, K, "lora_b NULL")


@pytest.mark.parametrize("T,K,os", [(1, 1024, (256,)), (8, 2560, (2560,)), (16, 384, (64, 64, 64)),
                                    (40, 512, (128,)), (300, 1024, (320, 64))])
def test_ternary_inputs_beyond_fp16_range(gpu, T, K, os):
    """x with values from 2^15 to 2e8 in a few tokens and chunks (the MFMA kernels stage x as fp16 hi/lo parts, whose
    range ends at 65504: those tokens' chunks take the scaled pass). On the MFMA kernels (T >= 5) every output is
    within the relative bound of the oracle's fp32 matmul, small values of the large tokens included; the rows kernel
    (T <= 4) follows the reference's decode arithmetic, whose cancellation adds a term in s sum |x|. The other tokens'
    outputs are unaffected. The north-star 2e-3 absolute bar is not applied: outputs here reach 1e7, where fp32 sums
    in another order differ by more."""
    torch, ctx, _ = gpu
    print(f"ternary large x T={T} K={K} os={os}", flush=True)
    mats, x, _, _ = make_case(0x7300 + T + K, T, K, os)
    x = x.copy()
    rng = np.random.default_rng(T + K)
    big_tokens = rng.choice(T, size=max(1, T // 4), replace=False)
    for t in big_tokens:
        cols = rng.choice(K, size=3, replace=False)
        x[t, cols] = np.array([1.0e5, -4.0e4, 7.0e4], np.float32) * (1 + 999 * (t % 3 == 0))
    x[big_tokens[0], -1] = 2.0e8
    got = run_gpu(torch, ctx, mats, x, K)
    ref = expected(mats, x, K)
    assert all(np.isfinite(g).all() for g in got)
    check(got, ref, mats, x, K, f"large x T={T} K={K}", abs_bar=False, cancel=T <= 4)
    small = np.setdiff1d(np.arange(T), big_tokens)
    if small.size:
        check([g[small] for g in got], [r[small] for r in ref], mats, x[small], K, "unaffected tokens")
    if T > 32:
        once = run_gpu(torch, ctx, mats, x, K, work=True)
        assert all(np.array_equal(a, b) for a, b in zip(got, once)), "split-once and in-place results differ"
