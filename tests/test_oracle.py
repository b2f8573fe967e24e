"""Pins the CPU oracle before it is trusted as the checker (CPU only).

The reference ships no kernel-level vectors for this path, and its shaders cannot be run here (no Rust,
glslc or Vulkan). Each oracle function is therefore pinned by what the mathematics fixes:
  - attention: float64 brute-force softmax(q k^T / 16) v over the causal window, plus invariants (split
    independence, L = 1, equal scores, a dominant key, causality, GQA head mapping, decode/verify equivalence);
  - fp16 storage: numpy's IEEE binary16 conversion, bit for bit, including subnormals, ties and overflow;
  - gate: sigmoid(0) = 1/2 exactly;
  - attn_prep: RMS-norm closed form, text-position mRoPE = standard rotate-half RoPE on 64 dims, sin/cos;
  - gate_rotate: the Sylvester Hadamard matrix (scipy) in float64.
"""
import numpy as np
import pytest
import scipy.linalg

import oracle
import workload

D = 256


def brute(q, kc, vc, off, gate=None, p16=False):
    """float64 closed form: out[t,h] = softmax_j<off+t+1 (q.k_j / 16) . v_j, then * sigmoid(gate). p16: each
    probability exp(s_j - max s) rounded to fp16 before both sums."""
    kf = oracle.f16_to_f32(kc).astype(np.float64)
    vf = oracle.f16_to_f32(vc).astype(np.float64)
    T, H = q.shape[0], q.shape[1]
    out = np.empty((T, H, D))
    for t in range(T):
        n = off + t + 1
        for h in range(H):
            kh = h // 4
            s = kf[:n, kh, :] @ q[t, h].astype(np.float64) / 16.0
            p = np.exp(s - s.max())
            if p16:
                p = p.astype(np.float16).astype(np.float64)
            out[t, h] = (p @ vf[:n, kh, :]) / p.sum()
    if gate is not None:
        out = out / (1.0 + np.exp(-gate.astype(np.float64)))
    return out


# ---------------------------------------------------------------------------------------------------------
# fp16 storage

def test_f32_to_f16_matches_ieee_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3.0),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),          # subnormal range of fp16
        (rng.standard_normal(20000) * 3e4).astype(np.float32),           # near overflow
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 * 0.9999],
                 dtype=np.float32),
    ])
    # exact ties between neighbouring fp16 values: (a + b) / 2 is an fp32 number
    a = np.arange(0x0001, 0x7BFF, 7, dtype=np.uint16)
    lo = a.view(np.float16).astype(np.float32)
    hi = (a + 1).view(np.float16).astype(np.float32)
    x = np.concatenate([x, (lo + hi) / np.float32(2.0), -(lo + hi) / np.float32(2.0)])
    ours = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):  # values past fp16's range are meant to become inf
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)
    nan = oracle.f32_to_f16(np.array([np.nan], dtype=np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def test_f16_to_f32_exact():
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    assert np.array_equal(np.isinf(ours), np.isinf(ref))


def test_append_rows():
    inp = workload.layer(5, T=3, off=4, H=4, KV=1)
    kc, vc = inp["kc"].copy(), inp["vc"].copy()
    oracle.append(inp["k_new"], inp["v_new"], kc, vc, 4)
    assert np.array_equal(kc[4:7], inp["k_new"].astype(np.float16).view(np.uint16))
    assert np.array_equal(vc[4:7], inp["v_new"].astype(np.float16).view(np.uint16))
    assert np.array_equal(kc[:4], inp["kc"][:4])


def test_generator_distribution():
    x = oracle.normal(123, 0, (400000,)).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert not np.array_equal(oracle.normal(123, 0, (8,)), oracle.normal(123, 1, (8,)))
    assert np.array_equal(oracle.normal(7, 3, (5,)), oracle.normal(7, 3, (5,)))
    r = oracle.rms_rows(oracle.normal(9, 0, (10, D)))
    assert np.allclose(np.sqrt((r.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-6)


# ---------------------------------------------------------------------------------------------------------
# attention

@pytest.mark.parametrize("T,off,H,KV,chunk", [
    (1, 0, 4, 1, 0), (1, 130, 8, 2, 0), (1, 511, 8, 2, 64), (5, 77, 8, 2, 0), (40, 100, 16, 4, 0),
    (24, 0, 4, 1, 16), (3, 600, 4, 1, 512)])
def test_attend_matches_float64_closed_form(T, off, H, KV, chunk):
    inp = workload.layer(11 + T + off, T=T, off=off, H=H, KV=KV)
    out, kc, vc = workload.expected(inp, chunk=chunk)
    ref = brute(inp["q"], kc, vc, off, inp["gate"])
    assert np.max(np.abs(out - ref)) < 2e-6


def test_attend_ungated_closed_form():
    inp = workload.layer(3, T=6, off=50, H=8, KV=2, gate=False)
    out, kc, vc = workload.expected(inp)
    assert np.max(np.abs(out - brute(inp["q"], kc, vc, 50))) < 2e-6


def test_split_count_does_not_change_result():
    inp = workload.layer(21, T=4, off=700, H=4, KV=1)
    outs = [workload.expected(inp, chunk=c)[0] for c in (16, 64, 512, 4096)]
    for o in outs[1:]:
        assert np.max(np.abs(o - outs[0])) < 1e-6


def test_single_key_returns_v_row_exactly():
    inp = workload.layer(4, T=1, off=0, H=8, KV=2, gate=False)
    out, kc, vc = workload.expected(inp)
    v = oracle.f16_to_f32(vc[0])  # [KV][256]
    for h in range(8):
        assert np.array_equal(out[0, h], v[h // 4])


def test_equal_scores_give_mean_of_v():
    inp = workload.layer(6, T=1, off=299, H=4, KV=1, gate=False)
    inp["q"][:] = 0.0
    out, kc, vc = workload.expected(inp)
    mean = oracle.f16_to_f32(vc[:300, 0]).astype(np.float64).mean(axis=0)
    assert np.max(np.abs(out[0] - mean)) < 1e-6


def test_dominant_key_selects_its_value():
    inp = workload.layer(8, T=1, off=199, H=4, KV=1, gate=False)
    kc0 = inp["kc"]
    j = 123
    kj = oracle.f16_to_f32(kc0[j, 0])
    inp["q"][0, 2] = 8.0 * kj  # score of key j = 8*|k_j|^2/16 = 128; the rest are far below
    out, kc, vc = workload.expected(inp)
    assert np.max(np.abs(out[0, 2] - oracle.f16_to_f32(vc[j, 0]))) < 1e-6


def test_causal_rows_ignore_later_keys():
    inp = workload.layer(12, T=6, off=30, H=4, KV=1)
    out, kc, vc = workload.expected(inp)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[33:] = oracle.f32_to_f16(oracle.normal(99, 0, kc2[33:].shape))
    vc2[33:] = oracle.f32_to_f16(oracle.normal(98, 0, vc2[33:].shape))
    out2 = oracle.attend(inp["q"], kc2, vc2, 30, inp["gate"])
    assert np.array_equal(out[:3], out2[:3])  # rows 0..2 see keys < 33 only
    assert not np.array_equal(out[3:], out2[3:])


def test_gqa_head_mapping():
    inp = workload.layer(13, T=2, off=40, H=8, KV=2)
    out, kc, vc = workload.expected(inp)
    kc2 = kc.copy()
    kc2[:, 1] = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(77, 0, (kc.shape[0], D))))
    out2 = oracle.attend(inp["q"], kc2, vc, 40, inp["gate"])
    assert np.array_equal(out[:, :4], out2[:, :4])     # heads 0..3 read kv head 0
    assert not np.any(np.all(out[:, 4:] == out2[:, 4:], axis=-1))


def test_rows_equal_single_row_decodes_bit_exactly():
    inp = workload.layer(14, T=7, off=300, H=8, KV=2)
    full, kc, vc = workload.expected(inp, chunk=64)
    rows, _, _ = workload.expected(inp, chunk=64, rows=range(7))
    assert np.array_equal(full, rows)


def test_gate_zero_halves_exactly():
    inp = workload.layer(15, T=3, off=20, H=4, KV=1)
    inp["gate"][:] = 0.0
    gated, kc, vc = workload.expected(inp)
    plain = oracle.attend(inp["q"], kc, vc, 20, None)
    assert np.array_equal(gated, plain * np.float32(0.5))


def test_gate_read_in_place_from_qproj_layout():
    """gate = q_proj output [T][H][512] + 256 (gate_rotate.comp:19-20), read through strides."""
    inp = workload.layer(16, T=3, off=9, H=8, KV=2)
    qp = oracle.normal(55, 0, (3, 8, 512))
    out_view, kc, vc = workload.expected(dict(inp, gate=qp[:, :, 256:]))
    out_copy = oracle.attend(inp["q"], kc, vc, 9, np.ascontiguousarray(qp[:, :, 256:]))
    assert np.array_equal(out_view, out_copy)


def test_ragged_equals_per_sequence():
    rng = np.random.default_rng(3)
    lens = rng.integers(1, 200, size=5).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    rows = int(lens.sum())
    kc = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(1, 2, (rows, 2, D))))
    vc = oracle.f32_to_f16(oracle.normal(1, 3, (rows, 2, D)))
    q = oracle.rms_rows(oracle.normal(1, 1, (5, 8, D)))
    z = oracle.normal(1, 6, (5, 8, D))
    out = oracle.decode_ragged(q, kc, vc, offs, lens, z)
    for i in range(5):
        o, n = offs[i], lens[i]
        ref = oracle.attend(q[i:i + 1], kc[o:o + n], vc[o:o + n], n - 1, z[i:i + 1])
        assert np.array_equal(out[i], ref[0])


def test_threads_do_not_change_bits():
    inp = workload.layer(17, T=9, off=600, H=8, KV=2)
    a = workload.expected(inp, nthreads=1)[0]
    b = workload.expected(inp, nthreads=4)[0]
    assert np.array_equal(a, b)


# ---------------------------------------------------------------------------------------------------------
# attn_prep

def _inv_freq(theta=1e7, rot=64):
    i = np.arange(rot // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), (2 * i).astype(np.float32) / np.float32(rot))).astype(np.float32)


def test_sincos_accuracy():
    xs = np.concatenate([np.linspace(-10, 10, 2001), np.linspace(0, 4096, 4001), [1e4, 3e4, 6e4]]).astype(np.float32)
    for x in xs:
        s, c = oracle.sincos(x)
        assert abs(s - np.sin(np.float64(x))) < 3e-7 * max(1.0, 1.0) + 2e-7
        assert abs(c - np.cos(np.float64(x))) < 5e-7


def test_prep_norm_and_text_rope():
    T, H, KV, off = 5, 8, 2, 3
    qp = oracle.normal(30, 0, (T, H, 512)) * np.float32(2.5)
    kp = oracle.normal(30, 1, (T, KV, D))
    vp = oracle.normal(30, 2, (T, KV, D))
    qn = (1.0 + 0.1 * oracle.normal(30, 3, (D,))).astype(np.float32)
    kn = (1.0 + 0.1 * oracle.normal(30, 4, (D,))).astype(np.float32)
    p = np.arange(100, 100 + T, dtype=np.int32)
    pos = np.stack([p, p, p])  # text tokens: all three mRoPE rows equal
    inv = _inv_freq()
    kc = np.zeros((off + T, KV, D), np.uint16)
    vc = np.zeros_like(kc)
    qout = oracle.prep(qp, kp, vp, qn, kn, pos, inv, kc, vc, off)

    def ref(x, w, t):
        x = x.astype(np.float64)
        y = x / np.sqrt((x ** 2).mean() + 1e-6) * w
        ang = p[t] * inv.astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        a, b = y[:32].copy(), y[32:64].copy()
        y[:32] = a * c - b * s
        y[32:64] = b * c + a * s
        return y

    for t in range(T):
        for h in range(H):
            assert np.max(np.abs(qout[t, h] - ref(qp[t, h, :256], qn, t))) < 2e-5
        for kh in range(KV):
            kref = ref(kp[t, kh], kn, t)
            got = oracle.f16_to_f32(kc[off + t, kh])
            assert np.max(np.abs(got - kref) / np.maximum(np.abs(kref), 1e-3)) < 1.5e-3
            assert np.array_equal(vc[off + t, kh], vp[t, kh].astype(np.float16).view(np.uint16))


def test_prep_mrope_sections_select_position_rows():
    """Interleaved mRoPE: pair i uses the h row if i%3==1 and i<33, the w row if i%3==2 and i<33, else t."""
    T, H, KV = 1, 4, 1
    qp = oracle.normal(31, 0, (T, H, 512))
    kp = oracle.normal(31, 1, (T, KV, D))
    vp = oracle.normal(31, 2, (T, KV, D))
    ones = np.ones(D, np.float32)
    inv = _inv_freq()
    pos = np.array([[7], [900], [40000]], np.int32)
    kc = np.zeros((1, KV, D), np.uint16)
    vc = np.zeros_like(kc)
    qout = oracle.prep(qp, kp, vp, ones, ones, pos, inv, kc, vc, 0)
    x = qp[0, 0, :256].astype(np.float64)
    y = x / np.sqrt((x ** 2).mean() + 1e-6)
    for i in range(32):
        sel = 1 if (i % 3 == 1 and i < 33) else (2 if (i % 3 == 2 and i < 33) else 0)
        ang = float(np.float32(pos[sel, 0]) * inv[i])  # the angle is an fp32 product (attn_prep.comp:52)
        assert abs(qout[0, 0, i] - (y[i] * np.cos(ang) - y[i + 32] * np.sin(ang))) < 3e-5
        assert abs(qout[0, 0, i + 32] - (y[i + 32] * np.cos(ang) + y[i] * np.sin(ang))) < 3e-5
    assert np.max(np.abs(qout[0, 0, 64:] - y[64:])) < 1e-5  # dims past ROT are only normalised


def test_gate_rotate_is_scaled_sylvester_hadamard():
    T, H = 2, 8
    W = H * 256
    attn = oracle.normal(40, 0, (T, W))
    qp = oracle.normal(40, 1, (T, 2 * W))
    signs = np.where(oracle.normal(40, 2, (W,)) > 0, 1.0, -1.0).astype(np.float32)
    xr = oracle.gate_rotate(attn, qp, signs)
    Hm = scipy.linalg.hadamard(512).astype(np.float64) / np.sqrt(512.0)
    for t in range(T):
        g = qp[t].reshape(H, 512)[:, 256:].reshape(W).astype(np.float64)
        x = attn[t].astype(np.float64) / (1.0 + np.exp(-g)) * signs
        ref = np.concatenate([Hm @ x[b:b + 512] for b in range(0, W, 512)])
        assert np.max(np.abs(xr[t] - ref)) < 2e-5


def test_p16_oracle_is_fp16_probabilities():
    """The perturbed oracle (the argmax tie margin's error budget) is the closed form with every probability
    rounded to fp16, and it differs from the exact oracle by about the fp16 rounding of P: more than fp32 noise,
    far less than the parity bar. One chunk covers every row's keys here, so the chunk max is the row max."""
    inp = workload.layer(321, T=3, off=40, H=4, KV=1)
    kc, vc = inp["kc"].copy(), inp["vc"].copy()
    oracle.append(inp["k_new"], inp["v_new"], kc, vc, inp["off"])
    exact = oracle.attend(inp["q"], kc, vc, 40, inp["gate"])
    pert = oracle.attend(inp["q"], kc, vc, 40, inp["gate"], p16=True)
    assert np.max(np.abs(pert - brute(inp["q"], kc, vc, 40, inp["gate"], p16=True))) < 2e-6
    d = np.max(np.abs(pert - exact))
    assert 1e-6 < d < 1e-3, d
    # ragged decodes carry the flag too
    offs, lens = np.array([0], np.int64), np.array([43], np.int32)
    r16 = oracle.decode_ragged(inp["q"][2:3], kc, vc, offs, lens, inp["gate"][2:3], p16=True)
    assert np.array_equal(r16[0], pert[2])


def test_argmax_tie_margin_comes_from_the_perturbed_reference():
    """With ref16 given, a reference row is a tie exactly when its top-2 projected gap is below
    3 sqrt(2) |ref16 - ref| of that row (and above the 1e-4 relative floor); the output under test plays no part."""
    rng = np.random.default_rng(5)
    H, T = 4, 4
    R = workload.projection(H)
    ref = rng.standard_normal((T, H, 256)).astype(np.float32)
    proj = ref.reshape(T, -1).astype(np.float64) @ R
    gap = np.sort(proj, axis=1)[:, -1] - np.sort(proj, axis=1)[:, -2]
    ref16 = ref.copy()
    e = rng.standard_normal(H * 256)
    e /= np.linalg.norm(e)
    scale = gap / (workload.TIE_SIGMAS * np.sqrt(2.0))  # |e16| at which a row's gap equals its margin
    for t, f in enumerate((2.0, 0.5, 1.2, 0.8)):  # rows 0 and 2: gap below the margin (ties); 1 and 3: above
        ref16[t] = (ref[t].reshape(-1) + f * scale[t] * e).reshape(H, 256)
    for out in (ref, ref + 1e-3 * rng.standard_normal(ref.shape).astype(np.float32)):
        bad, ties = workload.argmax_mismatches(out, ref, R, ref16)
        assert list(ties) == [0, 2] and len(bad) == 0


def test_argmax_check_flags_flips_and_excuses_only_ties():
    """The projected-argmax check of the GPU tests: a flip of a clear winner is reported, a flip between two
    columns whose reference values tie (within 1e-4 relative) is not, identical outputs report nothing."""
    rng = np.random.default_rng(3)
    H, T = 4, 6
    R = workload.projection(H)
    ref = rng.standard_normal((T, H, 256)).astype(np.float32)
    bad, ties = workload.argmax_mismatches(ref, ref, R)
    assert len(bad) == 0
    proj = ref.reshape(T, -1).astype(np.float64) @ R
    top = np.argmax(proj, axis=1)
    # row 0: push the runner-up far past the winner along its column direction -> a real mismatch
    second = np.argsort(proj[0])[-2]
    gap = proj[0, top[0]] - proj[0, second]
    col = R[:, second] / np.dot(R[:, second], R[:, second])
    out = ref.copy()
    out[0] = (ref[0].reshape(-1) + (gap + 1.0) * col).reshape(H, 256)
    bad, _ = workload.argmax_mismatches(out, ref, R)
    assert list(bad) == [0]
    # row 1: make the reference a tie between its two best columns, then let the output prefer the other one
    second = np.argsort(proj[1])[-2]
    d = R[:, top[1]] - R[:, second]
    shift = (proj[1, top[1]] - proj[1, second]) / np.dot(d, d)
    tie_ref = ref.copy()
    tie_ref[1] = (ref[1].reshape(-1) - shift * d * (1 - 1e-7)).reshape(H, 256)
    out = tie_ref.copy()
    out[1] = (tie_ref[1].reshape(-1) - 1e-6 * d).reshape(H, 256)
    bad, ties = workload.argmax_mismatches(out, tie_ref, R)
    assert 1 in ties and len(bad) == 0


# ---------------------------------------------------------------------------------------------------------
# Ternary linears (qmm3.comp order). Pinned by words written out by hand (the bit layout of qmv.glsl:1-2), a
# decoder that reads the codes out of each word's binary string, one-hot inputs (the column -> scale group map)
# and the LoRA / add closed forms.
def test_ternary_known_words():
    K, O = 128, 64
    w = np.full((O, K // 16), 0x55555555, np.uint32)  # every code 1: weight 0
    w[0, 0] = 0x00000000  # row 0, columns 0..15: code 0, weight -s
    w[1, 0] = 0xAAAAAAAA  # row 1, columns 0..15: code 2, weight +s
    w[2, 0] = 0x55555559  # row 2: column 0 code 1 (0), column 1 code 2 (+s), columns 2..15 code 1
    w[3, 7] = 0xD5555555  # row 3: column 127 = 16*7 + 15 has code 3 (+2s); bits 30-31 = 0b11
    w[4, 3] = 0x55555554  # row 4: column 48 code 0 (-s)
    s = oracle.f32_to_f16(np.full((O, 1), 0.5, np.float32))
    x = np.arange(1, K + 1, dtype=np.float32)[None, :]  # x[k] = k + 1
    y = oracle.ternary(w, s, x)[0]
    assert y[0] == -0.5 * np.sum(np.arange(1, 17))
    assert y[1] == 0.5 * np.sum(np.arange(1, 17))
    assert y[2] == 0.5 * 2.0
    assert y[3] == 2 * 0.5 * 128.0
    assert y[4] == -0.5 * 49.0
    assert not y[5:].any()


def decode_by_string(w, s):
    """float64 weights, reading code e of each word from its 32-character binary string (bits 2e, 2e+1)."""
    O, kw = w.shape
    sf = oracle.f16_to_f32(s).astype(np.float64)
    out = np.empty((O, kw * 16))
    for n in range(O):
        for j in range(kw):
            b = format(int(w[n, j]), "032b")
            for e in range(16):
                code = int(b[30 - 2 * e:32 - 2 * e], 2)
                out[n, 16 * j + e] = (code - 1) * sf[n, (16 * j + e) // 128]
    return out


def test_ternary_string_decoder():
    K, O, T = 256, 64, 3
    w, s, codes = workload.ternary_weights(0x7E01, O, K, code3=True)
    x = oracle.normal(0x7E01, 1, (T, K))
    ref = x.astype(np.float64) @ decode_by_string(w, s).T
    got = oracle.ternary(w, s, x)
    assert np.all(np.abs(got - ref) <= workload.ternary_tolerance(x, codes, s))
    # pack_codes is the inverse of the string decoder's reading
    dec = decode_by_string(w, oracle.f32_to_f16(np.ones((O, K // 128), np.float32)))
    assert np.array_equal(dec + 1, codes.astype(np.float64))


def test_ternary_scale_groups_one_hot():
    """x = e_k selects column k: y[n] = s[n, k // 128] * (code[n, k] - 1) exactly."""
    K, O = 384, 64
    w, s, codes = workload.ternary_weights(0x7E02, O, K, code3=True)
    cols = [0, 1, 15, 16, 127, 128, 200, 255, 256, 383]
    x = np.zeros((len(cols), K), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    got = oracle.ternary(w, s, x)
    sf = oracle.f16_to_f32(s)
    for i, k in enumerate(cols):
        assert np.array_equal(got[i], sf[:, k // 128] * (codes[:, k].astype(np.float32) - 1.0))


def test_ternary_add_and_lora():
    K, O, T, r = 128, 64, 2, 5
    w, s, codes = workload.ternary_weights(0x7E03, O, K)
    x = oracle.normal(0x7E03, 1, (T, K))
    y0 = oracle.normal(0x7E03, 2, (T, O))
    b = oracle.f32_to_f16(oracle.normal(0x7E03, 3, (O, r)))
    u = oracle.normal(0x7E03, 4, (T, r))
    plain = oracle.ternary(w, s, x)
    both = oracle.ternary(w, s, x, y=y0, lora_b=b, lora_u=u)
    lora = u.astype(np.float64) @ oracle.f16_to_f32(b).astype(np.float64).T
    assert np.max(np.abs(both - (y0 + plain + lora))) < 1e-5
    # all-zero codes: y = -s * sum(x) per scale group
    wz = np.zeros_like(w)
    got = oracle.ternary(wz, s, x)
    sf = oracle.f16_to_f32(s).astype(np.float64)
    assert np.max(np.abs(got - (-sf[:, 0][None, :] * x.astype(np.float64).sum(1)[:, None]))) < 1e-4


# norm_rotate: float64 closed form (RMS norm, then the Sylvester Hadamard matrix on each 512-block).
def test_norm_rotate_closed_form():
    T, Dm = 3, 1536
    h = oracle.normal(0x7E10, 0, (T, Dm)) * 3.0
    w = (1.0 + 0.1 * oracle.normal(0x7E10, 1, (Dm,))).astype(np.float32)
    signs = np.where(oracle.normal(0x7E10, 2, (Dm,)) > 0, 1.0, -1.0).astype(np.float32)
    xr, xn = oracle.norm_rotate(h, w, signs, want_xn=True)
    hd = h.astype(np.float64)
    r = 1.0 / np.sqrt((hd ** 2).mean(1, keepdims=True) + 1e-6)
    xn_ref = hd * r * w
    Hm = scipy.linalg.hadamard(512).astype(np.float64)
    xr_ref = np.concatenate([(xn_ref[:, b:b + 512] * signs[b:b + 512]) @ Hm.T for b in range(0, Dm, 512)], 1)
    xr_ref /= np.sqrt(512.0)
    assert np.max(np.abs(xn - xn_ref)) < 1e-5
    assert np.max(np.abs(xr - xr_ref)) < 2e-5
    # the rotation is orthogonal: row norms of xr equal those of signs * xn
    assert np.allclose(np.linalg.norm(xr.astype(np.float64), axis=1), np.linalg.norm(xn_ref, axis=1), rtol=1e-5)


@pytest.mark.parametrize("K", [512, 768, 2560, 4096])
def test_lora_closed_form(K):
    """u = A x in float64 (A the fp16 values): the LORA_ROW restatement agrees within fp32 rounding of its sums."""
    R, T = 7, 3
    A = oracle.f32_to_f16(oracle.normal(0x10A, 0, (R, K)) * 0.05)
    x = oracle.normal(0x10A, 1, (T, K))
    u = oracle.lora(A, x)
    prod = x.astype(np.float64)[:, None, :] * oracle.f16_to_f32(A).astype(np.float64)[None, :, :]
    ref = prod.sum(axis=2)
    assert np.all(np.abs(u - ref) <= 1e-6 * np.abs(prod).sum(axis=2) + 1e-12)


def test_lora_one_hot_rows_pick_columns():
    """Row r of A one-hot at column c_r gives u[t][r] = x[t][c_r] exactly, for columns in every thread's stride
    (4 i + 512 j) including past the last full 512-block of K = 768."""
    K = 768
    cols = [0, 1, 3, 4, 511, 512, 515, 700, 767]
    A = np.zeros((len(cols), K), np.uint16)
    for r, c in enumerate(cols):
        A[r, c] = oracle.f32_to_f16(np.array([1.0], np.float32))[0]
    x = oracle.normal(0x10B, 0, (2, K))
    u = oracle.lora(A, x)
    assert np.array_equal(u, x[:, cols])


def test_lora_gate_reads_the_gate_half():
    """gate_rotate's LoRA rows multiply A by attn * sigmoid(gate), the gate taken from the second half of every
    head's q_proj row (a restatement reading the q half, or skipping the sigmoid, fails)."""
    T, H = 2, 4
    W = H * D
    A = oracle.f32_to_f16(oracle.normal(0x10C, 0, (5, W)) * 0.05)
    attn = oracle.normal(0x10C, 1, (T, W))
    qp = oracle.normal(0x10C, 2, (T, H, 512))
    u = oracle.lora_gate(A, attn, qp)
    z = qp[:, :, D:].reshape(T, W).astype(np.float64)
    x = attn.astype(np.float64) / (1.0 + np.exp(-z))
    ref = x @ oracle.f16_to_f32(A).astype(np.float64).T
    assert np.max(np.abs(u - ref)) <= 1e-5 * np.max(np.abs(ref))
    wrong = (attn.astype(np.float64) / (1.0 + np.exp(-qp[:, :, :D].reshape(T, W)))) @ oracle.f16_to_f32(A).T
    assert np.max(np.abs(u - wrong)) > 1e-2
