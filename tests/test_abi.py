"""The C-ABI library: it loads, exports every symbol include/bonsai_attn.h declares, and its host-side argument
checks and workspace sizes behave as documented. CPU only: no call here touches a device."""
import ctypes
import os
import re

import pytest

from conftest import ROOT
from glimpse_language_amd import bonsai_attn as ba

HEADER = os.path.join(ROOT, "include", "bonsai_attn.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(ba.LIB_PATH):
        import importlib
        build = importlib.import_module("glimpse_language_amd.build")
        build.build()
    return ba.load()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:bn_status|size_t|void|const char\s*\*|int)\s+(bn_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert set(declared_functions()) == set(ba.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.bn_abi_version() == 6


def test_status_strings(lib):
    for s in range(5):
        assert lib.bn_status_str(s)


def fake(addr):
    return ctypes.c_void_p(addr)


def good_args(T=1, off=100, H=8, KV=2, cap=None):
    a = ba.AttnArgs()
    a.T, a.off, a.H, a.KV = T, off, H, KV
    a.cap = cap if cap is not None else off + T
    base = 0x100000
    a.q, a.q_ts, a.q_hs = base, H * 256, 256
    a.k_new, a.v_new = base + 0x1000, base + 0x2000
    a.kc, a.vc = base + 0x3000, base + 0x4000
    a.out, a.o_ts, a.o_hs = base + 0x5000, H * 256, 256
    a.gate, a.g_ts, a.g_hs = None, 0, 0
    need = ba.workspace_size(a)
    a.ws, a.ws_bytes = (base + 0x6000 if need else None), need
    return a


def test_check_accepts_good_shapes(lib):
    assert ba.check(good_args(), ba.KIND_DECODE) == ba.BN_OK
    assert ba.check(good_args(T=8, off=2048), ba.KIND_VERIFY) == ba.BN_OK
    assert ba.check(good_args(T=256, off=512), ba.KIND_PREFILL) == ba.BN_OK
    assert ba.check(good_args(T=4096, off=0, H=16, KV=4), ba.KIND_FORWARD) == ba.BN_OK
    assert ba.check(good_args(T=4, off=0), ba.KIND_APPEND) == ba.BN_OK


@pytest.mark.parametrize("mutate,kind,status", [
    (lambda a: setattr(a, "H", 6), ba.KIND_FORWARD, ba.BN_EINVAL),       # not 4:1
    (lambda a: setattr(a, "KV", 0), ba.KIND_FORWARD, ba.BN_EINVAL),
    (lambda a: setattr(a, "T", 0), ba.KIND_FORWARD, ba.BN_EINVAL),
    (lambda a: setattr(a, "cap", a.off + a.T - 1), ba.KIND_FORWARD, ba.BN_EINVAL),  # no room to append
    (lambda a: setattr(a, "T", 2), ba.KIND_DECODE, ba.BN_EINVAL),        # decode is one row
    (lambda a: (setattr(a, "T", 17), setattr(a, "cap", 200)), ba.KIND_VERIFY, ba.BN_EINVAL),
    (lambda a: setattr(a, "kc", 0x100008), ba.KIND_FORWARD, ba.BN_EINVAL),  # misaligned cache
    (lambda a: setattr(a, "v_new", None), ba.KIND_FORWARD, ba.BN_EINVAL),   # k_new without v_new
    (lambda a: setattr(a, "out", None), ba.KIND_FORWARD, ba.BN_EINVAL),
    (lambda a: setattr(a, "o_hs", 255), ba.KIND_FORWARD, ba.BN_EINVAL),
    (lambda a: setattr(a, "flags", 8), ba.KIND_FORWARD, ba.BN_EINVAL),
    (lambda a: (setattr(a, "k_new", None), setattr(a, "v_new", None)), ba.KIND_APPEND, ba.BN_EINVAL),
    (lambda a: setattr(a, "ws_bytes", a.ws_bytes - 16), ba.KIND_FORWARD, ba.BN_ENOWS),
    (lambda a: setattr(a, "ws", None), ba.KIND_FORWARD, ba.BN_ENOWS),
])
def test_check_rejects(lib, mutate, kind, status):
    a = good_args(T=1, off=5000)   # a decode over 5001 keys needs a workspace
    assert a.ws_bytes > 0
    mutate(a)
    assert ba.check(a, kind) == status
    assert ba.last_check_error()


def test_null_args_rejected(lib):
    assert lib.bn_attn_check(None, 0) == ba.BN_EINVAL
    assert lib.bn_ragged_check(None) == ba.BN_EINVAL
    assert lib.bn_attn_forward(None, None, None) == ba.BN_EINVAL


def test_workspace_sizes(lib):
    # a short decode is one split: no workspace
    assert ba.workspace_size(good_args(T=1, off=10)) == 0
    small = ba.workspace_size(good_args(T=1, off=1023))
    big = ba.workspace_size(good_args(T=1, off=32767))
    assert 0 < small < big
    r = ba.RaggedArgs()
    r.nseq, r.H, r.KV, r.max_len = 32, 16, 4, 32768
    sz = ba.workspace_size(r)
    assert sz > 0 and sz % 16 == 0
    # partial records of (m[4], l[4], acc[4][256]) floats per (sequence, kv head, split)
    assert sz % (4 * (8 + 4 * 256)) == 0


@pytest.mark.parametrize("T,H,KV,bound", [(8, 16, 4, 32768), (8, 16, 4, 131072), (12, 8, 2, 32768),
                                          (16, 16, 4, 131072), (2, 8, 2, 9000)])
def test_device_offset_workspace_stays_near_the_exact_one(lib, T, H, KV, bound):
    """With a device offset, `off` only bounds the rows' positions, and the workspace must cover every split count
    the kernels derive from a smaller offset. The kernels' chunk grows with the rows' total length, so that count
    stays near the exact one: the workspace is a small factor of the call at the bound without a device offset,
    not a linear function of the bound."""
    exact = good_args(T=T, off=bound - T, H=H, KV=KV)
    dyn = good_args(T=T, off=bound - T, H=H, KV=KV)
    dyn.dyn = 0x200000
    w_exact, w_dyn = ba.workspace_size(exact), ba.workspace_size(dyn)
    # the smallest offsets (a few keys per row) are covered too
    w_small = ba.workspace_size(good_args(T=T, off=0, H=H, KV=KV))
    assert w_dyn >= max(w_exact, w_small)
    assert w_dyn <= 4 * max(w_exact, 1 << 20), (w_dyn, w_exact)



def test_ragged_check(lib):
    r = ba.RaggedArgs()
    r.nseq, r.H, r.KV, r.max_len = 4, 8, 2, 100
    base = 0x200000
    r.q, r.q_ss, r.q_hs = base, 8 * 256, 256
    r.kc, r.vc = base + 0x1000, base + 0x2000
    r.kv_off, r.kv_len = base + 0x3000, base + 0x4000
    r.out, r.o_ss, r.o_hs = base + 0x5000, 8 * 256, 256
    need = ba.workspace_size(r)
    r.ws, r.ws_bytes = (base + 0x6000 if need else None), need
    assert ba.check(r) == ba.BN_OK
    r.kv_len = None
    assert ba.check(r) == ba.BN_EINVAL


def good_prep(T=4, off=10, H=8, KV=2):
    a = ba.PrepArgs()
    a.T, a.off, a.H, a.KV, a.cap = T, off, H, KV, off + T
    a.rot, a.s1, a.s2 = 64, 11, 11
    base = 0x300000
    a.qp, a.qp_ts, a.qp_hs = base, H * 512, 512
    a.kp, a.vp, a.q_norm, a.k_norm = base + 0x1000, base + 0x2000, base + 0x3000, base + 0x4000
    a.pos, a.inv_freq = base + 0x5000, base + 0x6000
    a.q, a.q_ts, a.q_hs = base + 0x7000, H * 256, 256
    a.kc, a.vc = base + 0x8000, base + 0x9000
    return a


@pytest.mark.parametrize("mutate", [
    lambda a: setattr(a, "H", 6),                                   # not 4:1
    lambda a: setattr(a, "T", 0),
    lambda a: setattr(a, "cap", a.off + a.T - 1),
    lambda a: setattr(a, "rot", 60),                                # not a multiple of 8
    lambda a: setattr(a, "rot", 264),
    lambda a: setattr(a, "pos", None),
    lambda a: setattr(a, "kc", 0x308008),                           # misaligned cache
    lambda a: setattr(a, "qp_hs", 510),
    lambda a: setattr(a, "flags", 2),
    lambda a: (setattr(a, "q", a.qp), setattr(a, "q_hs", 256)),     # in place with other strides
])
def test_prep_check(lib, mutate):
    a = good_prep()
    assert ba.check(a) == ba.BN_OK
    b = good_prep()
    b.q, b.q_ts, b.q_hs = b.qp, b.qp_ts, b.qp_hs                    # in place with the same strides is fine
    assert ba.check(b) == ba.BN_OK
    c = good_prep()
    c.rot, c.pos, c.inv_freq = 0, None, None                        # no rotary dims: no positions needed
    assert ba.check(c) == ba.BN_OK
    mutate(a)
    assert ba.check(a) == ba.BN_EINVAL
    assert ba.last_check_error()


@pytest.mark.parametrize("mutate", [
    lambda a: setattr(a, "H", 7),                                   # blocks of 512 are two heads
    lambda a: setattr(a, "H", 0),
    lambda a: setattr(a, "T", 0),
    lambda a: setattr(a, "signs", None),
    lambda a: setattr(a, "xr", 0x400002),
    lambda a: setattr(a, "g_hs", -1),
    lambda a: (setattr(a, "xr", a.attn), setattr(a, "x_ts", a.a_ts + 4)),
])
def test_rotate_check(lib, mutate):
    a = ba.RotateArgs()
    a.T, a.H = 3, 16
    base = 0x400000
    a.attn, a.a_ts = base, 16 * 256
    a.gate, a.g_ts, a.g_hs = base + 0x100000 + 256 * 4, 16 * 512, 512
    a.signs = base + 0x200000
    a.xr, a.x_ts = base + 0x300000, 16 * 256
    assert ba.check(a) == ba.BN_OK
    mutate(a)
    assert ba.check(a) == ba.BN_EINVAL
    assert ba.last_check_error()
    assert lib.bn_rotate_check(None) == ba.BN_EINVAL
    assert lib.bn_prep_check(None) == ba.BN_EINVAL


def layer_pair(T=1, off=100, H=8, KV=2):
    p = good_prep(T=T, off=off, H=H, KV=KV)
    a = ba.AttnArgs()
    a.T, a.off, a.H, a.KV, a.cap = T, off, H, KV, p.cap
    a.kc, a.vc = p.kc, p.vc
    a.out, a.o_ts, a.o_hs = 0x500000, H * 256, 256
    a.gate, a.g_ts, a.g_hs = p.qp + 1024, H * 512, 512
    probe = ba.AttnArgs()
    ctypes.pointer(probe)[0] = a
    probe.q, probe.q_ts, probe.q_hs, probe.k_new, probe.v_new = p.qp, p.qp_ts, p.qp_hs, p.kp, p.vp
    need = ba.workspace_size(probe)
    a.ws, a.ws_bytes = (0x600000 if need else None), need
    return p, a


def test_layer_check(lib):
    p, a = layer_pair()
    assert lib.bn_layer_check(p, a) == ba.BN_OK
    p.q = None                                   # q scratch not needed up to 16 rows
    assert lib.bn_layer_check(p, a) == ba.BN_OK
    p2, a2 = layer_pair(T=40, off=0)
    p2.q = None                                  # ... but needed for a prefill
    assert lib.bn_layer_check(p2, a2) == ba.BN_EINVAL
    p, a = layer_pair()
    a.q = p.qp                                   # the attention args take no q, k_new, v_new
    assert lib.bn_layer_check(p, a) == ba.BN_EINVAL
    p, a = layer_pair()
    a.off = 99                                   # both describe the same rows
    assert lib.bn_layer_check(p, a) == ba.BN_EINVAL
    p, a = layer_pair(T=1, off=5000)
    a.ws_bytes = 0                               # a multi-split decode needs the workspace
    assert lib.bn_layer_check(p, a) == ba.BN_ENOWS
    assert lib.bn_layer_check(None, a) == ba.BN_EINVAL
    assert lib.bn_attn_layer(None, None, None, None) == ba.BN_EINVAL


def kv_state(n_layers=3, KV=2, cap=100, length=40):
    s = ba.KvState()
    s.kc, s.vc = 0x700000, 0x800000
    s.n_layers, s.KV, s.cap, s.len = n_layers, KV, cap, length
    return s


def kv_section(n_layers, KV, length, body=None):
    import struct
    head = ba.KV_SECTION_MAGIC + struct.pack("<IIII", 1, n_layers, KV * 256, length)
    n = 2 * n_layers * length * KV * 256 * 2
    return head + (body if body is not None else bytes(n))


def test_kv_section_format_checks(lib):
    s = kv_state()
    assert lib.bn_kv_section_size(s) == 24 + 2 * 3 * 40 * 2 * 256 * 2
    good = kv_section(3, 2, 40)
    assert len(good) == lib.bn_kv_section_size(s)
    assert ba.kv_section_check(good, s) == (ba.BN_OK, 40)
    assert ba.kv_section_check(kv_section(3, 2, 100), s) == (ba.BN_OK, 100)    # up to the cache's cap
    assert ba.kv_section_check(kv_section(3, 2, 101), s)[0] == ba.BN_EINVAL    # more rows than the cache holds
    assert ba.kv_section_check(kv_section(2, 2, 40), s)[0] == ba.BN_EINVAL     # other layer count
    assert ba.kv_section_check(kv_section(3, 4, 40), s)[0] == ba.BN_EINVAL     # other row width
    assert ba.kv_section_check(good[:-2], s)[0] == ba.BN_EINVAL                # truncated
    assert ba.kv_section_check(good + b"\0", s)[0] == ba.BN_EINVAL             # trailing bytes
    assert ba.kv_section_check(b"BNSPFX01" + good[8:], s)[0] == ba.BN_EINVAL   # the reference's fp32 file magic
    bad_version = good[:8] + (2).to_bytes(4, "little") + good[12:]
    assert ba.kv_section_check(bad_version, s)[0] == ba.BN_EINVAL
    assert ba.kv_section_check(good[:10], s)[0] == ba.BN_EINVAL
    s.len = 101
    assert lib.bn_kv_section_size(s) == 0                                      # len beyond cap
    assert lib.bn_kv_copy(None, None, None, None) == ba.BN_EINVAL


def good_ternary(T=8, k=2560, os=(8192, 1024, 1024)):
    a = ba.TernaryArgs()
    a.T, a.k = T, k
    a.x, a.x_ts = 0x900000, k
    a.n_mats = len(os)
    for i, o in enumerate(os):
        base = 0x1000000 * (i + 1)
        a.mat[i].w, a.mat[i].s, a.mat[i].y = base, base + 0x800000, base + 0xC00000
        a.mat[i].o, a.mat[i].y_ts = o, o
    return a


@pytest.mark.parametrize("mutate", [
    lambda a: setattr(a, "k", 2500),                      # not a multiple of 128
    lambda a: setattr(a, "k", 0),
    lambda a: setattr(a, "n_mats", 0),
    lambda a: setattr(a, "n_mats", 4),
    lambda a: setattr(a, "T", 0),
    lambda a: setattr(a.mat[1], "o", 1000),               # not a multiple of 64
    lambda a: setattr(a.mat[0], "w", 0x1000008),          # W not 16-byte aligned
    lambda a: setattr(a, "x", 0x900004),                  # x not 16-byte aligned
    lambda a: setattr(a, "x_ts", 2562),                   # row stride not a multiple of 4
    lambda a: setattr(a, "x_ts", 2048),                   # row stride below k
    lambda a: setattr(a.mat[2], "y_ts", 512),             # output stride below o
    lambda a: setattr(a.mat[0], "y", 0),                  # missing output
    lambda a: setattr(a, "add", 2),
    lambda a: setattr(a, "lora_r", 8),                    # rank without u
    lambda a: setattr(a.mat[0], "lora_b", 0x1234000),     # B without a rank
])
def test_ternary_check(lib, mutate):
    assert lib.bn_ternary_check(good_ternary()) == ba.BN_OK
    assert lib.bn_ternary_check(good_ternary(T=1, k=128, os=(64,))) == ba.BN_OK
    a = good_ternary()
    a.lora_u, a.lora_us, a.lora_r = 0xA00000, 48, 16
    a.mat[1].lora_b = 0x2345000
    assert lib.bn_ternary_check(a) == ba.BN_OK
    a = good_ternary()
    mutate(a)
    assert lib.bn_ternary_check(a) == ba.BN_EINVAL
    assert "must" in ba.last_check_error() or "required" in ba.last_check_error() or "given" in ba.last_check_error()
    assert lib.bn_ternary_check(None) == ba.BN_EINVAL
    assert lib.bn_ternary_matmul(None, None, None) == ba.BN_EINVAL


def test_ternary_workspace(lib):
    """The optional workspace of T > 32 calls: 16 KB of split x per (64-token tile, 64-column chunk) plus a flag word;
    checked for size and 256-byte alignment only when the call would use it."""
    assert ba.ternary_workspace_size(32, 2560) == 0 and ba.ternary_workspace_size(1, 128) == 0
    assert ba.ternary_workspace_size(33, 256) == 4 * (16384 + 4)
    assert ba.ternary_workspace_size(4096, 2560) == 64 * 40 * (16384 + 4)
    need = ba.ternary_workspace_size(300, 2560)
    a = good_ternary(T=300)
    a.work, a.work_bytes = 0x40000000, need
    assert lib.bn_ternary_check(a) == ba.BN_OK
    a.work_bytes = need - 1
    assert lib.bn_ternary_check(a) == ba.BN_EINVAL and "work_bytes" in ba.last_check_error()
    a.work, a.work_bytes = 0x40000010, need
    assert lib.bn_ternary_check(a) == ba.BN_EINVAL and "aligned" in ba.last_check_error()
    a = good_ternary(T=8)
    a.work, a.work_bytes = 0x40000010, 1  # not used below 33 tokens
    assert lib.bn_ternary_check(a) == ba.BN_OK


@pytest.mark.parametrize("mutate", [
    lambda a: setattr(a, "d", 1000),          # not a multiple of 512
    lambda a: setattr(a, "T", 0),
    lambda a: setattr(a, "h", 0x900004),      # misaligned
    lambda a: setattr(a, "xr", 0),
    lambda a: setattr(a, "h_ts", 2048),       # stride below d
    lambda a: setattr(a, "xn_ts", 2561),      # stride not a multiple of 4
])
def test_norm_check(lib, mutate):
    def good():
        a = ba.NormArgs()
        a.T, a.d = 4, 2560
        a.h, a.h_ts, a.w, a.signs = 0x900000, 2560, 0xA00000, 0xB00000
        a.xn, a.xn_ts, a.xr, a.xr_ts = 0xC00000, 2560, 0xD00000, 2560
        return a
    assert lib.bn_norm_check(good()) == ba.BN_OK
    a = good()
    mutate(a)
    assert lib.bn_norm_check(a) == ba.BN_EINVAL
    assert lib.bn_norm_rotate(None, None, None) == ba.BN_EINVAL
