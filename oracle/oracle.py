"""ctypes binding of the CPU oracle (oracle/bn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by the cpu_baseline leg of
bench.py, always as the checker or the reported CPU baseline, never as the thing measured or shipped.
Functions and the reference code they restate are listed in oracle/bn_oracle.h.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbn_oracle.so")
D = 256

_lib = None


def build():
    subprocess.run(["make", "-C", HERE, "-s"], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    P, I, I64, U64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t
    L.bn_or_normal_f32.argtypes = [U64, U64, P, SZ]
    L.bn_or_normal_f32.restype = None
    L.bn_or_rms_rows.argtypes = [P, SZ, I]
    L.bn_or_rms_rows.restype = None
    L.bn_or_f32_to_f16_n.argtypes = [P, P, SZ]
    L.bn_or_f32_to_f16_n.restype = None
    L.bn_or_f16_to_f32_n.argtypes = [P, P, SZ]
    L.bn_or_f16_to_f32_n.restype = None
    L.bn_or_append.argtypes = [P, P, P, P, I, I, I]
    L.bn_or_append.restype = None
    L.bn_or_attend.argtypes = [I, I, I, I, I, P, I64, I64, P, P, P, I64, I64, P, I64, I64, I]
    L.bn_or_attend.restype = I
    L.bn_or_decode_ragged.argtypes = [I, I, I, I, P, I64, P, P, P, P, P, I64, P, I64, I]
    L.bn_or_decode_ragged.restype = I
    L.bn_or_attend_ex.argtypes = [I, I, I, I, I, P, I64, I64, P, P, P, I64, I64, P, I64, I64, I, I]
    L.bn_or_attend_ex.restype = I
    L.bn_or_decode_ragged_ex.argtypes = [I, I, I, I, P, I64, P, P, P, P, P, I64, P, I64, I, I]
    L.bn_or_decode_ragged_ex.restype = I
    L.bn_or_prep.argtypes = [P] * 10 + [I] * 7
    L.bn_or_prep.restype = None
    L.bn_or_sincos.argtypes = [ctypes.c_float, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
    L.bn_or_sincos.restype = None
    L.bn_or_gate_rotate.argtypes = [P, P, P, P, I, I]
    L.bn_or_gate_rotate.restype = None
    L.bn_or_norm_rotate.argtypes = [P, P, P, P, P, I, I]
    L.bn_or_norm_rotate.restype = None
    L.bn_or_ternary.argtypes = [P, P, P, I64, P, I64, I, I, I, I, P, P, I64, I, I]
    L.bn_or_ternary.restype = None
    L.bn_or_lora.argtypes = [P, P, I64, P, I64, I, I, I]
    L.bn_or_lora.restype = None
    L.bn_or_lora_gate.argtypes = [P, P, P, P, I64, I, I, I]
    L.bn_or_lora_gate.restype = None
    _lib = L
    return L


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def normal(seed, stream, shape):
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    lib().bn_or_normal_f32(seed, stream, _p(out), n)
    return out.reshape(shape)


def rms_rows(x):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().bn_or_rms_rows(_p(x), x.size // x.shape[-1], x.shape[-1])
    return x


def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().bn_or_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().bn_or_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def append(k_new, v_new, kc, vc, off):
    """kc/vc: uint16 [cap][KV][256] (modified in place)."""
    T, KV = k_new.shape[0], k_new.shape[1]
    assert off + T <= kc.shape[0]
    lib().bn_or_append(_p(np.ascontiguousarray(k_new, np.float32)), _p(np.ascontiguousarray(v_new, np.float32)),
                       _p(kc), _p(vc), T, off, KV)


def _strides(a):
    return [s // a.itemsize for s in a.strides]


def attend(q, kc, vc, off, gate=None, chunk=0, nthreads=0, p16=False):
    """Reference attention for T query rows at positions off..off+T-1 (cache rows [0, off+T) present).

    q, gate: float32 arrays [T][H][256] (any strides with unit innermost stride); kc, vc: uint16 fp16 bits
    [>=off+T][KV][256]. Returns out [T][H][256] float32. p16: the perturbed reference (every probability rounded
    to fp16 before both sums; not the reference's arithmetic) that sizes the argmax tie margins."""
    T, H = q.shape[0], q.shape[1]
    KV = kc.shape[1]
    assert q.strides[2] == 4 and kc.flags.c_contiguous and vc.flags.c_contiguous
    out = np.empty((T, H, D), dtype=np.float32)
    qs = _strides(q)
    gs = _strides(gate) if gate is not None else [0, 0, 0]
    if gate is not None:
        assert gate.dtype == np.float32 and gate.strides[2] == 4
    r = lib().bn_or_attend_ex(T, off, H, KV, chunk, _p(q), qs[0], qs[1], _p(kc), _p(vc), _p(gate), gs[0], gs[1],
                              _p(out), H * D, D, nthreads, int(bool(p16)))
    if r:
        raise ValueError("bn_or_attend rejected the shape")
    return out


def decode_ragged(q, kc, vc, kv_off, kv_len, gate=None, chunk=0, nthreads=0, p16=False):
    nseq, H = q.shape[0], q.shape[1]
    KV = kc.shape[1]
    q = np.ascontiguousarray(q, np.float32)
    gate = None if gate is None else np.ascontiguousarray(gate, np.float32)
    kv_off = np.ascontiguousarray(kv_off, np.int64)
    kv_len = np.ascontiguousarray(kv_len, np.int32)
    out = np.empty((nseq, H, D), dtype=np.float32)
    r = lib().bn_or_decode_ragged_ex(nseq, H, KV, chunk, _p(q), H * D, _p(kc), _p(vc), _p(kv_off), _p(kv_len),
                                     _p(gate), H * D, _p(out), H * D, nthreads, int(bool(p16)))
    if r:
        raise ValueError("bn_or_decode_ragged rejected the shape")
    return out


def prep(qp, kp, vp, qn, kn, pos, inv_freq, kc, vc, off, rot=64, s1=11, s2=11):
    """attn_prep: returns qout [T][H][256]; writes rows off..off+T-1 of kc/vc (uint16) in place."""
    T, H = qp.shape[0], qp.shape[1]
    KV = kp.shape[1]
    qout = np.empty((T, H, D), dtype=np.float32)
    args = [np.ascontiguousarray(a) for a in (qp, kp, vp, qn, kn)]
    pos = np.ascontiguousarray(pos, np.int32)
    inv_freq = np.ascontiguousarray(inv_freq, np.float32)
    lib().bn_or_prep(*[_p(a) for a in args], _p(pos), _p(inv_freq), _p(qout), _p(kc), _p(vc), T, off, H, KV, rot,
                     s1, s2)
    return qout


def sincos(x):
    s, c = ctypes.c_float(), ctypes.c_float()
    lib().bn_or_sincos(float(x), ctypes.byref(s), ctypes.byref(c))
    return s.value, c.value


def gate_rotate(attn, qp, signs):
    T, W = attn.shape
    xr = np.empty((T, W), dtype=np.float32)
    lib().bn_or_gate_rotate(_p(np.ascontiguousarray(attn, np.float32)), _p(np.ascontiguousarray(qp, np.float32)),
                            _p(np.ascontiguousarray(signs, np.float32)), _p(xr), T, W)
    return xr


def ternary(w, s, x, y=None, lora_b=None, lora_u=None, nthreads=0):
    """One ternary linear (qmm3.comp order): w uint32 [O][K/16], s uint16 fp16 [O][K/128], x float32 [T][K];
    y (float32 [T][O]) is added to when given (add = 1) and returned; lora_b uint16 [O][r], lora_u float32 [T][r]."""
    w = np.ascontiguousarray(w, np.uint32)
    s = np.ascontiguousarray(s, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    T, K = x.shape
    O = w.shape[0]
    assert w.shape == (O, K // 16) and s.shape == (O, K // 128)
    add = y is not None
    out = np.ascontiguousarray(y, np.float32).copy() if add else np.empty((T, O), np.float32)
    lr = 0 if lora_b is None else lora_b.shape[1]
    b = None if lora_b is None else np.ascontiguousarray(lora_b, np.uint16)
    u = None if lora_u is None else np.ascontiguousarray(lora_u, np.float32)
    lib().bn_or_ternary(_p(w), _p(s), _p(x), K, _p(out), O, T, K, O, int(add), _p(b), _p(u), lr, lr, nthreads)
    return out


def norm_rotate(h, w, signs, want_xn=False):
    """norm_rotate: returns xr [T][D] (and xn when want_xn)."""
    h = np.ascontiguousarray(h, np.float32)
    T, Dm = h.shape
    xr = np.empty_like(h)
    xn = np.empty_like(h) if want_xn else None
    lib().bn_or_norm_rotate(_p(h), _p(np.ascontiguousarray(w, np.float32)), _p(np.ascontiguousarray(signs, np.float32)),
                            _p(xn), _p(xr), T, Dm)
    return (xr, xn) if want_xn else xr


def lora(A, x):
    """LoRA down projection (rot.glsl:19-40 order): A uint16 fp16 bits [R][K], x float32 [T][K] -> u [T][R]."""
    A = np.ascontiguousarray(A, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    T, K = x.shape
    R = A.shape[0]
    assert A.shape[1] == K
    u = np.empty((T, R), np.float32)
    lib().bn_or_lora(_p(A), _p(x), K, _p(u), R, T, K, R)
    return u


def lora_gate(A, attn, qp):
    """gate_rotate's LoRA rows: x = attn * sigmoid(gate) with the gate at qp[t][h][256 + d]; attn [T][W]."""
    A = np.ascontiguousarray(A, np.uint16)
    attn = np.ascontiguousarray(attn, np.float32).reshape(attn.shape[0], -1)
    T, W = attn.shape
    qp = np.ascontiguousarray(qp, np.float32).reshape(T, 2 * W)
    R = A.shape[0]
    u = np.empty((T, R), np.float32)
    lib().bn_or_lora_gate(_p(A), _p(attn), _p(qp), _p(u), R, T, W, R)
    return u
