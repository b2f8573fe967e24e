"""Seeded synthetic attention-layer inputs shared by the tests (drawn with the oracle's generator).

Q and K rows are RMS-normalised N(0,1) samples (post-QK-norm, post-RoPE), V and the gate logits are N(0,1);
K/V cache rows are stored as fp16. Seeds follow the workload list: 0xB0A5A100 + workload index.
"""
import numpy as np

import oracle

D = 256
SEED_BASE = 0xB0A5A100
PROJ_SEED = 0xA5A5

# (name, H, KV, T, off): the single-GPU workloads the library is checked on
WORKLOADS = {
    "decode_1k": dict(H=8, KV=2, T=1, off=1023),       # one query vs 1024 keys (incl. the new one)
    "prefill_prefix": dict(H=8, KV=2, T=256, off=512),  # user turn over a cached 512-row prefix
    "verify_8": dict(H=8, KV=2, T=8, off=2048),         # 8 drafts vs 2048 cached rows
    "prefill_4k": dict(H=16, KV=4, T=4096, off=0),      # 4B-scale 4096-row causal prefill
}


def layer(seed, T, off, H, KV, cap=None, gate=True):
    """Inputs of one attention call. kc/vc rows [off, off+T) hold filler the call overwrites."""
    cap = cap or off + T
    q = oracle.rms_rows(oracle.normal(seed, 1, (T, H, D)))
    kc = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(seed, 2, (cap, KV, D))))
    vc = oracle.f32_to_f16(oracle.normal(seed, 3, (cap, KV, D)))
    k_new = oracle.rms_rows(oracle.normal(seed, 4, (T, KV, D)))
    v_new = oracle.normal(seed, 5, (T, KV, D))
    z = oracle.normal(seed, 6, (T, H, D)) if gate else None
    return dict(q=q, kc=kc, vc=vc, k_new=k_new, v_new=v_new, gate=z, T=T, off=off, H=H, KV=KV, cap=cap)


def expected(inp, chunk=0, nthreads=0, rows=None, p16=False):
    """Oracle output after appending k_new/v_new; rows (optional) selects query rows (decode-equivalent); p16: the
    perturbed oracle (probabilities rounded to fp16) that sizes the argmax tie margin."""
    kc, vc = inp["kc"].copy(), inp["vc"].copy()
    oracle.append(inp["k_new"], inp["v_new"], kc, vc, inp["off"])
    if rows is None:
        out = oracle.attend(inp["q"], kc, vc, inp["off"], inp["gate"], chunk, nthreads, p16)
        return out, kc, vc
    outs = []
    for t in rows:
        g = None if inp["gate"] is None else inp["gate"][t:t + 1]
        outs.append(oracle.attend(inp["q"][t:t + 1], kc, vc, inp["off"] + t, g, chunk, nthreads, p16)[0])
    return np.stack(outs), kc, vc


# Prefill parity shapes (T, off, H, KV, gate): single-tile q-tiles, tails, offsets that are not multiples of 32 (rows
# with no key in the second half of a split key range), head counts with KV not dividing 8, 1 and 2 key tiles per
# group.
PREFILL_SHAPES = [(2, 0, 4, 1, True), (31, 0, 8, 2, True), (32, 0, 4, 1, False), (33, 0, 4, 1, True),
                  (50, 20, 8, 2, True), (64, 64, 8, 2, True), (100, 37, 12, 3, True), (130, 500, 16, 4, False),
                  (257, 0, 8, 2, True), (256, 512, 8, 2, True), (96, 1000, 4, 1, True), (3, 2000, 8, 2, True)]


def prefill_shape_input(T, off, H, KV, gate, q16):
    """Inputs of one prefill parity shape; q16: query rows rounded to fp16 first (the values an fp16-q kernel
    multiplies). The seeds give references with at most tie_cap(T) argmax ties (pinned on the CPU)."""
    inp = layer(6002 + 7 * T + off, T=T, off=off, H=H, KV=KV, gate=gate)
    if q16:
        inp["q"] = inp["q"].astype(np.float16).astype(np.float32)
    return inp


def projection(H):
    return oracle.normal(PROJ_SEED, 0, (H * D, 128)).astype(np.float64)


def projected_argmax(out, R):
    T = out.shape[0]
    return np.argmax(out.reshape(T, -1).astype(np.float64) @ R, axis=1)


# A reference row counts as a tie when its two best projected values lie closer than an fp16 implementation of the
# same sums can move them. The error budget is fixed apart from the output under test: ref16, the oracle with every
# probability rounded to fp16 before both sums (the rounding every fp16-MFMA kernel applies to P), gives the row's
# error e16 = ref16 - ref. A projection column of R (N(0,1) weights) moves by N(0, |e|^2) under an output error e,
# the difference of two columns by sqrt(2) |e|, so the margin is max(TIE_REL of the top value, TIE_SIGMAS sqrt(2)
# |e16|): a kernel whose error is of e16's size swaps a row outside it with probability below 0.14%. A kernel with a
# larger error (a dropped term, a wrong scale) shows as max-abs error or as swaps in rows outside the margin; the
# tests also bound the number of tie rows to max(2, rows / 100).
TIE_REL = 1e-4
TIE_SIGMAS = 3.0


def tie_cap(rows):
    return max(2, rows // 100)


def argmax_mismatches(out, ref, R, ref16=None):
    """Rows whose projected argmax differs between `out` and `ref`, and the reference rows that are ties (top-2
    margin below the tie margin above; TIE_REL alone without ref16) and therefore not compared. Returns (mismatched
    rows, tie rows)."""
    T = ref.shape[0]
    r = ref.reshape(T, -1).astype(np.float64)
    o = out.reshape(T, -1).astype(np.float64)
    pr = r @ R
    po = o @ R
    top2 = np.sort(pr, axis=1)[:, -2:]
    margin = TIE_REL * np.abs(top2[:, 1])
    if ref16 is not None:
        e16 = np.linalg.norm(ref16.reshape(T, -1).astype(np.float64) - r, axis=1)
        margin = np.maximum(margin, TIE_SIGMAS * np.sqrt(2.0) * e16)
    tie = (top2[:, 1] - top2[:, 0]) < margin
    diff = np.argmax(po, axis=1) != np.argmax(pr, axis=1)
    return np.nonzero(diff & ~tie)[0], np.nonzero(tie)[0]


# ---- ternary projections ------------------------------------------------------------------------------------
def ternary_weights(seed, O, K, code3=False):
    """Packed ternary weights: codes uniform in {0, 1, 2} (and 3 when code3, weight 2 * scale), 16 per uint32 with
    code e of word j (column 16j + e) at bits [2e, 2e + 2); fp16 scales |N(0,1)| * 0.02 + 0.005 per 128 columns."""
    u = oracle.normal(seed, 7, (O, K))
    hi = 4 if code3 else 3
    codes = np.floor((np.tanh(u) * 0.5 + 0.5) * hi).clip(0, hi - 1).astype(np.uint32)
    w = pack_codes(codes)
    s = oracle.f32_to_f16(np.abs(oracle.normal(seed, 8, (O, K // 128))) * 0.02 + 0.005)
    return w, s, codes


def pack_codes(codes):
    """[O, K] codes 0..3 -> [O, K/16] uint32."""
    O, K = codes.shape
    c = codes.reshape(O, K // 16, 16).astype(np.uint32)
    return np.bitwise_or.reduce(c << (2 * np.arange(16, dtype=np.uint32)), axis=2).astype(np.uint32)


def ternary_tolerance(x, codes, s):
    """Per-output bound for comparing two fp32 evaluations of x W^T: 2e-5 * ||(x_k w_k)_k||_2 + 1e-6. fp32 sums of K
    products differ by about 2^-24 sqrt(K) of that norm (3e-6 at K = 2560); rounding x to fp16 alone would move them
    by about 2^-12 of it (2.4e-4), so a path that dropped x's low half fails."""
    w = (codes.astype(np.float64) - 1.0) * np.repeat(oracle.f16_to_f32(s).astype(np.float64), 128, axis=1)
    n2 = (x.astype(np.float64) ** 2) @ (w ** 2).T
    return 2e-5 * np.sqrt(n2) + 1e-6
