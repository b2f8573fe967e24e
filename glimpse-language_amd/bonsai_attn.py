"""ctypes binding of include/bonsai_attn.h (the C ABI of libbonsai_attn.so).

This is the binding a Python caller (tests, benchmark) uses; the Rust runtime binds the same symbols through
an `extern "C"` block. Device memory and streams come from the caller: here torch tensors on a ROCm device
supply raw pointers (torch is plumbing only; the library itself never sees a torch type).

The product path has no fallback: if the library is missing, `load()` raises.
"""
import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libbonsai_attn.so")

D = 256
VERIFY_MAX = 16

BN_OK, BN_EINVAL, BN_ENOWS, BN_ELAUNCH, BN_EDEVICE = 0, 1, 2, 3, 4
BN_Q_F16 = 1
KIND_FORWARD, KIND_DECODE, KIND_VERIFY, KIND_PREFILL, KIND_APPEND = 0, 1, 2, 3, 4

# every symbol include/bonsai_attn.h declares
EXPORTS = (
    "bn_ctx_create", "bn_ctx_destroy", "bn_status_str", "bn_ctx_last_error", "bn_abi_version",
    "bn_attn_workspace_size", "bn_ragged_workspace_size", "bn_attn_check", "bn_ragged_check",
    "bn_workspace_clear", "bn_attn_forward", "bn_attn_decode", "bn_attn_verify", "bn_attn_prefill",
    "bn_attn_append", "bn_attn_decode_ragged", "bn_prep_check", "bn_rotate_check", "bn_attn_prep",
    "bn_gate_rotate", "bn_attn_layer", "bn_layer_check", "bn_kv_copy", "bn_kv_section_size", "bn_kv_section_save",
    "bn_kv_section_check", "bn_kv_section_load", "bn_ternary_check", "bn_ternary_matmul", "bn_norm_check",
    "bn_norm_rotate", "bn_attn_decode_ragged_noalloc", "bn_ternary_workspace_size", "bn_dyn_overflow",
)
KV_SECTION_MAGIC = b"BNKVF16\0"
KV_SECTION_HEADER = 24


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_uint32), ("off", ctypes.c_uint32), ("H", ctypes.c_uint32), ("KV", ctypes.c_uint32),
        ("cap", ctypes.c_uint32), ("flags", ctypes.c_uint32),
        ("q", ctypes.c_void_p), ("q_ts", ctypes.c_int64), ("q_hs", ctypes.c_int64),
        ("k_new", ctypes.c_void_p), ("v_new", ctypes.c_void_p),
        ("kc", ctypes.c_void_p), ("vc", ctypes.c_void_p),
        ("gate", ctypes.c_void_p), ("g_ts", ctypes.c_int64), ("g_hs", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("o_ts", ctypes.c_int64), ("o_hs", ctypes.c_int64),
        ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_size_t),
        ("signs", ctypes.c_void_p),
        ("dyn", ctypes.c_void_p),
        ("lora_a", ctypes.c_void_p), ("lora_u", ctypes.c_void_p), ("lora_us", ctypes.c_int64),
        ("lora_r", ctypes.c_uint32),
    ]


class RaggedArgs(ctypes.Structure):
    _fields_ = [
        ("nseq", ctypes.c_uint32), ("H", ctypes.c_uint32), ("KV", ctypes.c_uint32), ("max_len", ctypes.c_uint32),
        ("q", ctypes.c_void_p), ("q_ss", ctypes.c_int64), ("q_hs", ctypes.c_int64),
        ("k_new", ctypes.c_void_p), ("v_new", ctypes.c_void_p),
        ("kc", ctypes.c_void_p), ("vc", ctypes.c_void_p),
        ("kv_off", ctypes.c_void_p), ("kv_len", ctypes.c_void_p),
        ("gate", ctypes.c_void_p), ("g_ss", ctypes.c_int64), ("g_hs", ctypes.c_int64),
        ("out", ctypes.c_void_p), ("o_ss", ctypes.c_int64), ("o_hs", ctypes.c_int64),
        ("ws", ctypes.c_void_p), ("ws_bytes", ctypes.c_size_t),
        ("signs", ctypes.c_void_p),
    ]


class PrepArgs(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_uint32), ("off", ctypes.c_uint32), ("H", ctypes.c_uint32), ("KV", ctypes.c_uint32),
        ("cap", ctypes.c_uint32), ("flags", ctypes.c_uint32), ("rot", ctypes.c_uint32), ("s1", ctypes.c_uint32),
        ("s2", ctypes.c_uint32),
        ("qp", ctypes.c_void_p), ("qp_ts", ctypes.c_int64), ("qp_hs", ctypes.c_int64),
        ("kp", ctypes.c_void_p), ("vp", ctypes.c_void_p), ("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p),
        ("pos", ctypes.c_void_p), ("inv_freq", ctypes.c_void_p),
        ("q", ctypes.c_void_p), ("q_ts", ctypes.c_int64), ("q_hs", ctypes.c_int64),
        ("kc", ctypes.c_void_p), ("vc", ctypes.c_void_p),
        ("dyn", ctypes.c_void_p),
    ]


class RotateArgs(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_uint32), ("H", ctypes.c_uint32),
        ("attn", ctypes.c_void_p), ("a_ts", ctypes.c_int64),
        ("gate", ctypes.c_void_p), ("g_ts", ctypes.c_int64), ("g_hs", ctypes.c_int64),
        ("signs", ctypes.c_void_p),
        ("xr", ctypes.c_void_p), ("x_ts", ctypes.c_int64),
        ("lora_a", ctypes.c_void_p), ("lora_u", ctypes.c_void_p), ("lora_us", ctypes.c_int64),
        ("lora_r", ctypes.c_uint32),
    ]


class KvState(ctypes.Structure):
    _fields_ = [
        ("kc", ctypes.c_void_p), ("vc", ctypes.c_void_p),
        ("n_layers", ctypes.c_uint32), ("KV", ctypes.c_uint32), ("cap", ctypes.c_uint32), ("len", ctypes.c_uint32),
    ]


_lib = None


class TernaryMat(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("y", ctypes.c_void_p), ("lora_b", ctypes.c_void_p),
        ("o", ctypes.c_uint32), ("y_ts", ctypes.c_int64),
    ]


class TernaryArgs(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_uint32), ("k", ctypes.c_uint32), ("x", ctypes.c_void_p), ("x_ts", ctypes.c_int64),
        ("n_mats", ctypes.c_uint32), ("add", ctypes.c_uint32), ("mat", TernaryMat * 3),
        ("lora_u", ctypes.c_void_p), ("lora_us", ctypes.c_int64), ("lora_r", ctypes.c_uint32),
        ("work", ctypes.c_void_p), ("work_bytes", ctypes.c_uint64),
    ]


class NormArgs(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_uint32), ("d", ctypes.c_uint32), ("h", ctypes.c_void_p), ("h_ts", ctypes.c_int64),
        ("w", ctypes.c_void_p), ("signs", ctypes.c_void_p), ("xn", ctypes.c_void_p), ("xn_ts", ctypes.c_int64),
        ("xr", ctypes.c_void_p), ("xr_ts", ctypes.c_int64),
        ("lora_a", ctypes.c_void_p), ("lora_u", ctypes.c_void_p), ("lora_us", ctypes.c_int64),
        ("lora_r", ctypes.c_uint32),
    ]


def load(path=LIB_PATH):
    """Loads the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with glimpse-language_amd/build.py")
    lib = ctypes.CDLL(path)
    P = ctypes.c_void_p
    lib.bn_ctx_create.argtypes = [ctypes.c_int, ctypes.POINTER(P)]
    lib.bn_ctx_create.restype = ctypes.c_int
    lib.bn_ctx_destroy.argtypes = [P]
    lib.bn_ctx_destroy.restype = None
    lib.bn_status_str.argtypes = [ctypes.c_int]
    lib.bn_status_str.restype = ctypes.c_char_p
    lib.bn_ctx_last_error.argtypes = [P]
    lib.bn_ctx_last_error.restype = ctypes.c_char_p
    lib.bn_abi_version.argtypes = []
    lib.bn_abi_version.restype = ctypes.c_int
    lib.bn_dyn_overflow.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    lib.bn_dyn_overflow.restype = ctypes.c_int
    lib.bn_attn_workspace_size.argtypes = [ctypes.POINTER(AttnArgs)]
    lib.bn_attn_workspace_size.restype = ctypes.c_size_t
    lib.bn_ragged_workspace_size.argtypes = [ctypes.POINTER(RaggedArgs)]
    lib.bn_ragged_workspace_size.restype = ctypes.c_size_t
    lib.bn_attn_check.argtypes = [ctypes.POINTER(AttnArgs), ctypes.c_int]
    lib.bn_attn_check.restype = ctypes.c_int
    lib.bn_ragged_check.argtypes = [ctypes.POINTER(RaggedArgs)]
    lib.bn_ragged_check.restype = ctypes.c_int
    lib.bn_workspace_clear.argtypes = [P, P, P, ctypes.c_size_t]
    lib.bn_workspace_clear.restype = ctypes.c_int
    for name in ("bn_attn_forward", "bn_attn_decode", "bn_attn_verify", "bn_attn_prefill", "bn_attn_append"):
        f = getattr(lib, name)
        f.argtypes = [P, P, ctypes.POINTER(AttnArgs)]
        f.restype = ctypes.c_int
    for name in ("bn_attn_decode_ragged", "bn_attn_decode_ragged_noalloc"):
        f = getattr(lib, name)
        f.argtypes = [P, P, ctypes.POINTER(RaggedArgs)]
        f.restype = ctypes.c_int
    lib.bn_prep_check.argtypes = [ctypes.POINTER(PrepArgs)]
    lib.bn_prep_check.restype = ctypes.c_int
    lib.bn_rotate_check.argtypes = [ctypes.POINTER(RotateArgs)]
    lib.bn_rotate_check.restype = ctypes.c_int
    lib.bn_attn_prep.argtypes = [P, P, ctypes.POINTER(PrepArgs)]
    lib.bn_attn_prep.restype = ctypes.c_int
    lib.bn_gate_rotate.argtypes = [P, P, ctypes.POINTER(RotateArgs)]
    lib.bn_gate_rotate.restype = ctypes.c_int
    lib.bn_attn_layer.argtypes = [P, P, ctypes.POINTER(PrepArgs), ctypes.POINTER(AttnArgs)]
    lib.bn_attn_layer.restype = ctypes.c_int
    lib.bn_layer_check.argtypes = [ctypes.POINTER(PrepArgs), ctypes.POINTER(AttnArgs)]
    lib.bn_layer_check.restype = ctypes.c_int
    K = ctypes.POINTER(KvState)
    lib.bn_kv_copy.argtypes = [P, P, K, K]
    lib.bn_kv_copy.restype = ctypes.c_int
    lib.bn_kv_section_size.argtypes = [K]
    lib.bn_kv_section_size.restype = ctypes.c_size_t
    lib.bn_kv_section_save.argtypes = [P, P, K, P, ctypes.c_size_t]
    lib.bn_kv_section_save.restype = ctypes.c_int
    lib.bn_kv_section_check.argtypes = [P, ctypes.c_size_t, K, ctypes.POINTER(ctypes.c_uint32)]
    lib.bn_kv_section_check.restype = ctypes.c_int
    lib.bn_kv_section_load.argtypes = [P, P, P, ctypes.c_size_t, K, ctypes.POINTER(ctypes.c_uint32)]
    lib.bn_kv_section_load.restype = ctypes.c_int
    lib.bn_ternary_check.argtypes = [ctypes.POINTER(TernaryArgs)]
    lib.bn_ternary_check.restype = ctypes.c_int
    lib.bn_ternary_matmul.argtypes = [P, P, ctypes.POINTER(TernaryArgs)]
    lib.bn_ternary_matmul.restype = ctypes.c_int
    lib.bn_ternary_workspace_size.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    lib.bn_ternary_workspace_size.restype = ctypes.c_size_t
    lib.bn_norm_check.argtypes = [ctypes.POINTER(NormArgs)]
    lib.bn_norm_check.restype = ctypes.c_int
    lib.bn_norm_rotate.argtypes = [P, P, ctypes.POINTER(NormArgs)]
    lib.bn_norm_rotate.restype = ctypes.c_int
    _lib = lib
    return lib


class BonsaiAttnError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{msg} (status {status})")
        self.status = status


def last_check_error():
    return load().bn_ctx_last_error(None).decode()


class Context:
    """bn_ctx on one device. Calls are ordered on the given stream (default: torch's current stream)."""

    def __init__(self, device=0):
        lib = load()
        h = ctypes.c_void_p()
        st = lib.bn_ctx_create(device, ctypes.byref(h))
        if st != BN_OK:
            raise BonsaiAttnError(st, f"bn_ctx_create({device}) failed: {lib.bn_status_str(st).decode()}")
        self.h = h
        self.lib = lib
        self.device = device

    def close(self):
        if self.h:
            self.lib.bn_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def error(self):
        return self.lib.bn_ctx_last_error(self.h).decode()

    def dyn_overflow(self):
        """Reads and clears the device's overflow flag (bn_dyn_overflow): True if a call since the last read found
        a device offset above its host bound (it then attended as at the bound and appended nothing)."""
        flag = ctypes.c_int(0)
        self._check(self.lib.bn_dyn_overflow(self.h, ctypes.byref(flag)), "bn_dyn_overflow")
        return bool(flag.value)

    def _stream(self, stream):
        if stream is not None:
            return ctypes.c_void_p(int(stream))
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    def _check(self, st, what):
        if st != BN_OK:
            raise BonsaiAttnError(st, f"{what}: {self.error()}")

    def call(self, name, args, stream=None):
        f = getattr(self.lib, name)
        st = f(self.h, self._stream(stream), ctypes.byref(args))
        self._check(st, name)

    def workspace_clear(self, ws_ptr, nbytes, stream=None):
        st = self.lib.bn_workspace_clear(self.h, self._stream(stream), ctypes.c_void_p(ws_ptr), nbytes)
        self._check(st, "bn_workspace_clear")


def _ptr(t):
    return None if t is None else t.data_ptr()


def set_lora(a, lora):
    """Fills an args struct's LoRA-A fields from lora = (A [R][K] fp16/int16, U [T][R] float32 with unit inner stride),
    or clears them (None)."""
    if lora is None:
        a.lora_a, a.lora_u, a.lora_us, a.lora_r = None, None, 0, 0
        return a
    A, U = lora
    a.lora_a, a.lora_u = _ptr(A), _ptr(U)
    a.lora_us = U.stride(0)
    a.lora_r = A.shape[0]
    return a


def attn_args(T, off, H, KV, cap, q, kc, vc, out, k_new=None, v_new=None, gate=None, ws=None, flags=0,
              q_strides=None, g_strides=None, o_strides=None, signs=None, dyn=None):
    """bn_attn_args from tensors. q [T][H][256] (or explicit strides), gate/out likewise; kc/vc fp16 caches
    viewed as int16/float16 tensors; ws a byte tensor or None."""
    a = AttnArgs()
    a.T, a.off, a.H, a.KV, a.cap, a.flags = T, off, H, KV, cap, flags
    a.q = _ptr(q)
    a.q_ts, a.q_hs = q_strides if q_strides else (H * D, D)
    a.k_new, a.v_new = _ptr(k_new), _ptr(v_new)
    a.kc, a.vc = _ptr(kc), _ptr(vc)
    a.gate = _ptr(gate)
    a.g_ts, a.g_hs = g_strides if g_strides else (H * D, D)
    a.out = _ptr(out)
    a.o_ts, a.o_hs = o_strides if o_strides else (H * D, D)
    a.ws = _ptr(ws)
    a.ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    a.signs = _ptr(signs)
    a.dyn = _ptr(dyn)
    return a


def ragged_args(nseq, H, KV, max_len, q, kc, vc, kv_off, kv_len, out, k_new=None, v_new=None, gate=None,
                ws=None, signs=None):
    a = RaggedArgs()
    a.nseq, a.H, a.KV, a.max_len = nseq, H, KV, max_len
    a.q, a.q_ss, a.q_hs = _ptr(q), H * D, D
    a.k_new, a.v_new = _ptr(k_new), _ptr(v_new)
    a.kc, a.vc = _ptr(kc), _ptr(vc)
    a.kv_off, a.kv_len = _ptr(kv_off), _ptr(kv_len)
    a.gate, a.g_ss, a.g_hs = _ptr(gate), H * D, D
    a.out, a.o_ss, a.o_hs = _ptr(out), H * D, D
    a.ws = _ptr(ws)
    a.ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    a.signs = _ptr(signs)
    return a


def workspace_size(args):
    lib = load()
    if isinstance(args, RaggedArgs):
        return lib.bn_ragged_workspace_size(ctypes.byref(args))
    return lib.bn_attn_workspace_size(ctypes.byref(args))


def check(args, kind=KIND_FORWARD):
    lib = load()
    if isinstance(args, RaggedArgs):
        return lib.bn_ragged_check(ctypes.byref(args))
    if isinstance(args, PrepArgs):
        return lib.bn_prep_check(ctypes.byref(args))
    if isinstance(args, RotateArgs):
        return lib.bn_rotate_check(ctypes.byref(args))
    return lib.bn_attn_check(ctypes.byref(args), kind)


class Workspace:
    """A caller-owned, zero-initialised device workspace that grows on demand (torch uint8 tensor)."""

    def __init__(self, ctx, device="cuda"):
        self.ctx = ctx
        self.device = device
        self.buf = None

    def get(self, nbytes):
        import torch
        if nbytes == 0:
            return None
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self.device)
            self.ctx.workspace_clear(self.buf.data_ptr(), self.buf.numel())
        return self.buf


_KIND_FN = {KIND_FORWARD: "bn_attn_forward", KIND_DECODE: "bn_attn_decode", KIND_VERIFY: "bn_attn_verify",
            KIND_PREFILL: "bn_attn_prefill", KIND_APPEND: "bn_attn_append"}


def bind(ctx, name, *structs, stream=None):
    """A zero-argument callable that issues library entry `name` on `stream` with argument structs built once
    (as a compiled caller would), checking the status."""
    f = getattr(ctx.lib, name)
    st = ctx._stream(stream)
    refs = [ctypes.byref(x) for x in structs]

    def call():
        ctx._check(f(ctx.h, st, *refs), name)
    call.structs = structs
    return call


def attention(ctx, ws, q, kc, vc, off, out=None, k_new=None, v_new=None, gate=None, kind=KIND_FORWARD,
              stream=None, q_strides=None, g_strides=None, signs=None, dyn=None, lora=None):
    """One attention-layer call: append k_new/v_new at [off, off+T), attend causally, gate (and, with signs,
    rotate: out is then o_proj's input).

    q: [T, H, 256] fp32, or fp16 (passed with BN_Q_F16); kc/vc: [cap, KV, 256] fp16 (torch.float16 or int16
    view); out: [T, H, 256] fp32; signs: [H * 256] fp32 +-1; dyn: a uint32/int32 device tensor holding the
    offset read at run time (off is then its upper bound).
    """
    a, out = attention_args(ctx, ws, q, kc, vc, off, out, k_new, v_new, gate, q_strides, g_strides, signs, dyn)
    set_lora(a, lora)
    ctx.call(_KIND_FN[kind], a, stream)
    return out


def attention_args(ctx, ws, q, kc, vc, off, out=None, k_new=None, v_new=None, gate=None, q_strides=None,
                   g_strides=None, signs=None, dyn=None):
    """The bn_attn_args of an attention() call (workspace attached) and its output tensor."""
    import torch
    T, H = q.shape[0], q.shape[1]
    cap, KV = kc.shape[0], kc.shape[1]
    if out is None:
        out = torch.empty((T, H, D), dtype=torch.float32, device=q.device)
    flags = BN_Q_F16 if q.dtype == torch.float16 else 0
    a = attn_args(T, off, H, KV, cap, q, kc, vc, out, k_new, v_new, gate, None, flags, q_strides, g_strides,
                  signs=signs, dyn=dyn)
    need = workspace_size(a)
    buf = ws.get(need) if ws is not None else None
    a.ws = _ptr(buf)
    a.ws_bytes = 0 if buf is None else buf.numel()
    return a, out


def decode_ragged(ctx, ws, q, kc, vc, kv_off, kv_len, max_len, out=None, k_new=None, v_new=None, gate=None,
                  stream=None, signs=None):
    a, out = decode_ragged_args(ctx, ws, q, kc, vc, kv_off, kv_len, max_len, out, k_new, v_new, gate, signs)
    ctx.call("bn_attn_decode_ragged", a, stream)
    return out


def decode_ragged_noalloc(ctx, q, kc, vc, kv_off, kv_len, max_len, out=None, k_new=None, v_new=None, gate=None,
                          stream=None, signs=None):
    """bn_attn_decode_ragged_noalloc: decode_ragged() with the split partials in the library's own per-device array
    instead of a workspace (no allocation in the call)."""
    a, out = decode_ragged_args(ctx, None, q, kc, vc, kv_off, kv_len, max_len, out, k_new, v_new, gate, signs)
    ctx.call("bn_attn_decode_ragged_noalloc", a, stream)
    return out


NOALLOC_SCRATCH_BYTES = 16 << 20


def decode_ragged_args(ctx, ws, q, kc, vc, kv_off, kv_len, max_len, out=None, k_new=None, v_new=None, gate=None,
                       signs=None):
    """The bn_ragged_args of a decode_ragged() call (workspace attached) and its output tensor."""
    import torch
    nseq, H = q.shape[0], q.shape[1]
    KV = kc.shape[1]
    if out is None:
        out = torch.empty((nseq, H, D), dtype=torch.float32, device=q.device)
    a = ragged_args(nseq, H, KV, max_len, q, kc, vc, kv_off, kv_len, out, k_new, v_new, gate, signs=signs)
    need = workspace_size(a)
    buf = ws.get(need) if ws is not None else None
    a.ws = _ptr(buf)
    a.ws_bytes = 0 if buf is None else buf.numel()
    return a, out


def prep_args(qp, kp, vp, q_norm, k_norm, pos, inv_freq, q, kc, vc, off, rot=64, s1=11, s2=11, dyn=None):
    """bn_prep_args from tensors. qp: [T, H, >=256] with unit stride in the last dim (the q_proj output
    [T, H, 512] as it is); kp/vp [T, KV, 256]; pos int32 [3, T]; q [T, H, 256] fp32 or fp16 (BN_Q_F16)."""
    import torch
    a = PrepArgs()
    T, H = qp.shape[0], qp.shape[1]
    a.T, a.off, a.H, a.KV, a.cap = T, off, H, kc.shape[1], kc.shape[0]
    a.flags = BN_Q_F16 if q.dtype == torch.float16 else 0
    a.rot, a.s1, a.s2 = rot, s1, s2
    a.qp, a.qp_ts, a.qp_hs = _ptr(qp), qp.stride(0), qp.stride(1)
    a.kp, a.vp, a.q_norm, a.k_norm = _ptr(kp), _ptr(vp), _ptr(q_norm), _ptr(k_norm)
    a.pos, a.inv_freq = _ptr(pos), _ptr(inv_freq)
    a.q, a.q_ts, a.q_hs = _ptr(q), q.stride(0), q.stride(1)
    a.kc, a.vc = _ptr(kc), _ptr(vc)
    a.dyn = _ptr(dyn)
    return a


def attn_prep(ctx, qp, kp, vp, q_norm, k_norm, pos, inv_freq, kc, vc, off, rot=64, s1=11, s2=11, q=None,
              q_dtype=None, stream=None, dyn=None):
    """attn_prep: writes normed, rotated q (returned) and the fp16 K/V cache rows [off, off + T)."""
    import torch
    T, H = qp.shape[0], qp.shape[1]
    if q is None:
        q = torch.empty((T, H, D), dtype=q_dtype or torch.float32, device=qp.device)
    ctx.call("bn_attn_prep", prep_args(qp, kp, vp, q_norm, k_norm, pos, inv_freq, q, kc, vc, off, rot, s1, s2, dyn),
             stream)
    return q


def rotate_args(attn, signs, xr, gate=None, lora=None):
    """bn_rotate_args from tensors: attn/xr [T, W] or [T, H, 256] (unit stride inside a row), gate a view
    [T, H, 256] with unit stride in the last dim (e.g. qp[:, :, 256:]) or None."""
    a = RotateArgs()
    T = attn.shape[0]
    W = signs.numel()
    a.T, a.H = T, W // D
    a.attn, a.a_ts = _ptr(attn), attn.stride(0)
    a.gate = _ptr(gate)
    a.g_ts, a.g_hs = (gate.stride(0), gate.stride(1)) if gate is not None else (0, 0)
    a.signs = _ptr(signs)
    a.xr, a.x_ts = _ptr(xr), xr.stride(0)
    return set_lora(a, lora)


def gate_rotate(ctx, attn, signs, gate=None, xr=None, stream=None, lora=None):
    """gate_rotate: xr = H_512 (attn * sigmoid(gate) * signs) / sqrt(512) per 512-element block (returned); with
    lora = (A, U) also U[t] = A (attn * sigmoid(gate))[t]."""
    import torch
    if xr is None:
        xr = torch.empty((attn.shape[0], signs.numel()), dtype=torch.float32, device=attn.device)
    ctx.call("bn_gate_rotate", rotate_args(attn, signs, xr, gate, lora), stream)
    return xr


def attention_layer(ctx, ws, qp, kp, vp, q_norm, k_norm, pos, inv_freq, kc, vc, off, gate=None, signs=None,
                    out=None, q=None, rot=64, s1=11, s2=11, stream=None, dyn=None, lora=None):
    """bn_attn_layer: attn_prep + attention (+ gate, + rotation with signs) in one call. qp [T, H, >=256] raw q
    rows (q_proj's output as it is), kp/vp [T, KV, 256] raw; gate a [T, H, 256] view with unit stride in the
    last dim (e.g. qp[:, :, 256:]); q: scratch [T, H, 256] for T > 16 (allocated when None)."""
    p, a, out = attention_layer_args(ctx, ws, qp, kp, vp, q_norm, k_norm, pos, inv_freq, kc, vc, off, gate, signs,
                                     out, q, rot, s1, s2, dyn)
    set_lora(a, lora)
    st = ctx.lib.bn_attn_layer(ctx.h, ctx._stream(stream), ctypes.byref(p), ctypes.byref(a))
    ctx._check(st, "bn_attn_layer")
    return out


def attention_layer_args(ctx, ws, qp, kp, vp, q_norm, k_norm, pos, inv_freq, kc, vc, off, gate=None, signs=None,
                         out=None, q=None, rot=64, s1=11, s2=11, dyn=None):
    """The (bn_prep_args, bn_attn_args, out) of an attention_layer call, for callers that issue it repeatedly."""
    import torch
    T, H = qp.shape[0], qp.shape[1]
    KV, cap = kc.shape[1], kc.shape[0]
    if out is None:
        out = torch.empty((T, H, D), dtype=torch.float32, device=qp.device)
    if q is None and T > VERIFY_MAX:
        q = torch.empty((T, H, D), dtype=torch.float32, device=qp.device)
    p = PrepArgs()
    p.T, p.off, p.H, p.KV, p.cap = T, off, H, KV, cap
    p.flags = BN_Q_F16 if (q is not None and q.dtype == torch.float16) else 0
    p.rot, p.s1, p.s2 = rot, s1, s2
    p.qp, p.qp_ts, p.qp_hs = _ptr(qp), qp.stride(0), qp.stride(1)
    p.kp, p.vp, p.q_norm, p.k_norm = _ptr(kp), _ptr(vp), _ptr(q_norm), _ptr(k_norm)
    p.pos, p.inv_freq = _ptr(pos), _ptr(inv_freq)
    p.q = _ptr(q)
    p.q_ts, p.q_hs = (q.stride(0), q.stride(1)) if q is not None else (0, 0)
    p.kc, p.vc = _ptr(kc), _ptr(vc)
    p.dyn = _ptr(dyn)
    g_strides = (gate.stride(0), gate.stride(1)) if gate is not None else None
    a = attn_args(T, off, H, KV, cap, None, kc, vc, out, None, None, gate, None, 0, (0, 0), g_strides, None,
                  signs=signs, dyn=dyn)
    probe = attn_args(T, off, H, KV, cap, qp, kc, vc, out, kp, vp, gate, None, 0, (qp.stride(0), qp.stride(1)),
                      g_strides, None, signs=signs, dyn=dyn)
    need = workspace_size(probe)
    buf = ws.get(need) if ws is not None else None
    a.ws = _ptr(buf)
    a.ws_bytes = 0 if buf is None else buf.numel()
    return p, a, out


def kv_state(kc, vc, length):
    """bn_kv_state of caches kc/vc shaped [n_layers, cap, KV, 256] (fp16 or int16 views) with `length` rows used."""
    st = KvState()
    st.kc, st.vc = _ptr(kc), _ptr(vc)
    st.n_layers, st.cap, st.KV = kc.shape[0], kc.shape[1], kc.shape[2]
    st.len = length
    return st


def kv_copy(ctx, src, dst, stream=None):
    """encode_copy_state's KV part: rows [0, src.len) of every layer from state src into state dst."""
    st = ctx.lib.bn_kv_copy(ctx.h, ctx._stream(stream), ctypes.byref(src), ctypes.byref(dst))
    ctx._check(st, "bn_kv_copy")


def kv_section_save(ctx, state, stream=None):
    """The KV section of a saved prefix (bytes)."""
    n = load().bn_kv_section_size(ctypes.byref(state))
    if n == 0:
        raise BonsaiAttnError(BN_EINVAL, "bad KV state")
    buf = ctypes.create_string_buffer(n)
    st = ctx.lib.bn_kv_section_save(ctx.h, ctx._stream(stream), ctypes.byref(state), buf, n)
    ctx._check(st, "bn_kv_section_save")
    return buf.raw


def kv_section_check(data, state):
    """(status, len) of a KV section against a state, on the host."""
    n = ctypes.c_uint32(0)
    st = load().bn_kv_section_check(data, len(data), ctypes.byref(state), ctypes.byref(n))
    return st, n.value


def kv_section_load(ctx, data, state, stream=None):
    """Loads a KV section into state's caches; returns its len."""
    n = ctypes.c_uint32(0)
    st = ctx.lib.bn_kv_section_load(ctx.h, ctx._stream(stream), data, len(data), ctypes.byref(state), ctypes.byref(n))
    ctx._check(st, "bn_kv_section_load")
    return n.value


def ternary_workspace_size(T, K):
    """bn_ternary_workspace_size: bytes of the optional workspace of a T x K call (0 for T <= 32)."""
    return load().bn_ternary_workspace_size(T, K)


def ternary_workspace(x):
    """A device workspace (uint8 tensor) for bn_ternary_matmul over x [T, K], or None when the call uses none."""
    n = ternary_workspace_size(x.shape[0], x.shape[1])
    if not n:
        return None
    import torch
    return torch.empty(n, dtype=torch.uint8, device=x.device)


def ternary_args(x, mats, add=False, lora_u=None, lora_r=0, work=None):
    """bn_ternary_args: x [T, K] float32 (unit stride inside a row); mats: up to three (w, s, y) or
    (w, s, y, lora_b) with w int32/uint32 [O, K/16], s fp16/int16 [O, K/128], y [T, O] float32; work: an optional
    workspace from ternary_workspace(x) (T > 32: x is then split once per call)."""
    a = TernaryArgs()
    a.T, a.k = x.shape[0], x.shape[1]
    a.x, a.x_ts = _ptr(x), x.stride(0)
    a.n_mats = len(mats)
    a.add = int(bool(add))
    for i, m in enumerate(mats):
        w, sc, y = m[0], m[1], m[2]
        lb = m[3] if len(m) > 3 else None
        a.mat[i].w, a.mat[i].s, a.mat[i].y, a.mat[i].lora_b = _ptr(w), _ptr(sc), _ptr(y), _ptr(lb)
        a.mat[i].o = w.shape[0]
        a.mat[i].y_ts = y.stride(0)
    a.lora_u = _ptr(lora_u)
    a.lora_us = lora_u.stride(0) if lora_u is not None else 0
    a.lora_r = lora_r
    a.work = _ptr(work)
    a.work_bytes = work.numel() * work.element_size() if work is not None else 0
    return a


def ternary_matmul(ctx, x, mats, add=False, lora_u=None, lora_r=0, stream=None, work=None):
    """bn_ternary_matmul: y_i (+)= x W_i^T (+ LoRA) for each (w, s, y[, lora_b]) in mats; y tensors are written."""
    ctx.call("bn_ternary_matmul", ternary_args(x, mats, add, lora_u, lora_r, work), stream)


def norm_args(h, w, signs, xr, xn=None, lora=None):
    a = NormArgs()
    a.T, a.d = h.shape[0], h.shape[1]
    a.h, a.h_ts = _ptr(h), h.stride(0)
    a.w, a.signs = _ptr(w), _ptr(signs)
    a.xn, a.xn_ts = _ptr(xn), xn.stride(0) if xn is not None else 0
    a.xr, a.xr_ts = _ptr(xr), xr.stride(0)
    return set_lora(a, lora)


def norm_rotate(ctx, h, w, signs, xr=None, xn=None, stream=None, lora=None):
    """norm_rotate: xr = FWHT-512(signs * rmsnorm(h) * w) / sqrt(512) per block (returned); xn = rmsnorm(h) * w;
    with lora = (A, U) also U[t] = A xn[t]."""
    import torch
    if xr is None:
        xr = torch.empty_like(h)
    ctx.call("bn_norm_rotate", norm_args(h, w, signs, xr, xn, lora), stream)
    return xr
