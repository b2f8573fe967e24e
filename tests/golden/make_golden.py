"""Writes the golden vectors of the attention path: tests/golden/*.npz (inputs and expected outputs).

The reference ships no kernel-level vectors for attention, so these are produced by the oracle
(oracle/bn_oracle.c, a restatement of attn_split.comp + attn_combine.comp + gate_rotate.comp) and, before
they are written, checked against an independent float64 brute-force softmax attention (max-abs 2e-6).
Each file holds: q, gate (fp32, absent for the ungated cases), kc, vc (fp16 bits as uint16; rows [0, off)
are the cache, rows [off, off+T) the filler the call overwrites), k_new, v_new (fp32), out (fp32, computed
after the append) and shape = (T, off, H, KV). Ragged files hold kv_off/kv_len and shape = (nseq, H, KV);
k_new[i] goes to row kv_off[i] + kv_len[i] - 1. The cache after the call is fp16(k_new), fp16(v_new) in
those rows (nearest even) and is not stored.

    python tests/golden/make_golden.py     (deterministic: the same bytes on every run)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle  # noqa: E402
import workload  # noqa: E402

D = 256

# name: (seed, T, off, H, KV, gate)
CASES = {
    "decode_8q2kv_L200": (0xB0A5A100, 1, 199, 8, 2, True),
    "decode_16q4kv_L65_nogate": (0xB0A5A110, 1, 64, 16, 4, False),
    "verify_8q2kv_T8_off120": (0xB0A5A102, 8, 120, 8, 2, True),
    "prefill_8q2kv_T24_off40_nogate": (0xB0A5A101, 24, 40, 8, 2, False),
}
RAGGED = {"ragged_16q4kv_4seq": (0xB0A5A104, 4, 16, 4, 1, 60)}


def brute(q, kc, vc, off, gate):
    kf = oracle.f16_to_f32(kc).astype(np.float64)
    vf = oracle.f16_to_f32(vc).astype(np.float64)
    T, H = q.shape[0], q.shape[1]
    out = np.empty((T, H, D))
    for t in range(T):
        n = off + t + 1
        for h in range(H):
            s = kf[:n, h // 4, :] @ q[t, h].astype(np.float64) / 16.0
            p = np.exp(s - s.max())
            out[t, h] = (p @ vf[:n, h // 4, :]) / p.sum()
    if gate is not None:
        out = out / (1.0 + np.exp(-gate.astype(np.float64)))
    return out


def make_case(seed, T, off, H, KV, gate):
    inp = workload.layer(seed, T=T, off=off, H=H, KV=KV, gate=gate)
    out, kc, vc = workload.expected(inp)
    err = np.max(np.abs(out - brute(inp["q"], kc, vc, off, inp["gate"])))
    assert err < 2e-6, err
    d = dict(q=inp["q"], kc=inp["kc"], vc=inp["vc"], k_new=inp["k_new"], v_new=inp["v_new"], out=out,
             shape=np.array([T, off, H, KV], np.int64))
    if gate:
        d["gate"] = inp["gate"]
    return d


def make_ragged(seed, nseq, H, KV, lo, hi):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=nseq).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    rows = int(lens.sum())
    kc = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(seed, 2, (rows, KV, D))))
    vc = oracle.f32_to_f16(oracle.normal(seed, 3, (rows, KV, D)))
    q = oracle.rms_rows(oracle.normal(seed, 1, (nseq, H, D)))
    k_new = oracle.rms_rows(oracle.normal(seed, 4, (nseq, KV, D)))
    v_new = oracle.normal(seed, 5, (nseq, KV, D))
    z = oracle.normal(seed, 6, (nseq, H, D))
    kc_after, vc_after = kc.copy(), vc.copy()
    for i in range(nseq):
        r = offs[i] + lens[i] - 1
        kc_after[r] = oracle.f32_to_f16(k_new[i])
        vc_after[r] = oracle.f32_to_f16(v_new[i])
    out = oracle.decode_ragged(q, kc_after, vc_after, offs, lens, z)
    for i in range(nseq):
        o, n = offs[i], lens[i]
        ref = brute(q[i:i + 1], kc_after[o:o + n], vc_after[o:o + n], n - 1, z[i:i + 1])
        assert np.max(np.abs(out[i] - ref[0])) < 2e-6
    return dict(q=q, gate=z, kc=kc, vc=vc, k_new=k_new, v_new=v_new, out=out, kv_off=offs, kv_len=lens,
                shape=np.array([nseq, H, KV], np.int64))


def main():
    for name, args in CASES.items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **make_case(*args))
        print("wrote", name)
    for name, args in RAGGED.items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **make_ragged(*args))
        print("wrote", name)


if __name__ == "__main__":
    main()
