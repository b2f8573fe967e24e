"""Prefix-state snapshots of the attention layers on the GPU: bn_kv_copy (encode_copy_state's KV part,
model.rs:1072-1086) and the KV section save/load (state_parts + save_prefix / load_prefix, model.rs:1088-1099,
mod.rs:492-578), in the fp16 format of include/bonsai_attn.h.

Checked: the saved bytes are the header and the used fp16 rows in the documented order (compared with the
rows built on the host); a load into a cache of another capacity restores exactly those rows and leaves the
rest untouched; a copy between states moves exactly the used rows; attention over a restored cache is
bit-identical to attention over the original; a section that fails its check leaves the device untouched.
"""
import struct

import numpy as np
import pytest

import oracle
import workload
from test_gpu_attn import to_dev as attn_to_dev
from glimpse_language_amd import bonsai_attn as ba

pytestmark = pytest.mark.gpu
D = 256


def make_caches(seed, n_layers, cap, KV, length):
    kc = np.zeros((n_layers, cap, KV, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :length] = oracle.f32_to_f16(oracle.rms_rows(oracle.normal(seed, 0, (n_layers, length, KV, D))))
    vc[:, :length] = oracle.f32_to_f16(oracle.normal(seed, 1, (n_layers, length, KV, D)))
    return kc, vc


def dev16(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).cuda()


def host16(t):
    return t.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("n_layers,KV,cap,length", [(3, 2, 300, 257), (2, 4, 64, 1), (1, 1, 10, 0)])
def test_section_round_trip(gpu, n_layers, KV, cap, length):
    torch, ctx, _ = gpu
    kc, vc = make_caches(0xE000 + cap, n_layers, cap, KV, length)
    d_kc, d_vc = dev16(torch, kc), dev16(torch, vc)
    data = ba.kv_section_save(ctx, ba.kv_state(d_kc, d_vc, length))
    head = ba.KV_SECTION_MAGIC + struct.pack("<IIII", 1, n_layers, KV * D, length)
    body = kc[:, :length].tobytes() + vc[:, :length].tobytes()
    assert data == head + body
    # into a cache with room for more rows: the used rows come back, the rest is untouched
    cap2 = cap + 37
    kc2 = np.full((n_layers, cap2, KV, D), 0x3C00, np.uint16)  # fp16 1.0 everywhere
    vc2 = kc2.copy()
    d_kc2, d_vc2 = dev16(torch, kc2), dev16(torch, vc2)
    assert ba.kv_section_load(ctx, data, ba.kv_state(d_kc2, d_vc2, 0)) == length
    got_k, got_v = host16(d_kc2), host16(d_vc2)
    assert np.array_equal(got_k[:, :length], kc[:, :length]) and np.array_equal(got_v[:, :length], vc[:, :length])
    assert np.all(got_k[:, length:] == 0x3C00) and np.all(got_v[:, length:] == 0x3C00)


def test_copy_between_states(gpu):
    torch, ctx, _ = gpu
    n_layers, KV, length = 4, 2, 150
    kc, vc = make_caches(0xE100, n_layers, 400, KV, length)
    d_kc, d_vc = dev16(torch, kc), dev16(torch, vc)
    d_kc3 = torch.zeros((n_layers, length, KV, D), dtype=torch.int16, device="cuda")  # a snapshot sized to the prefix
    d_vc3 = torch.zeros_like(d_kc3)
    ba.kv_copy(ctx, ba.kv_state(d_kc, d_vc, length), ba.kv_state(d_kc3, d_vc3, 0))
    d_kc4 = torch.zeros((n_layers, 300, KV, D), dtype=torch.int16, device="cuda")  # ... and back into a live state
    d_vc4 = torch.zeros_like(d_kc4)
    ba.kv_copy(ctx, ba.kv_state(d_kc3, d_vc3, length), ba.kv_state(d_kc4, d_vc4, 0))
    torch.cuda.synchronize()
    assert np.array_equal(host16(d_kc3), kc[:, :length]) and np.array_equal(host16(d_vc3), vc[:, :length])
    assert np.array_equal(host16(d_kc4)[:, :length], kc[:, :length])
    assert np.array_equal(host16(d_vc4)[:, :length], vc[:, :length])
    assert not host16(d_kc4)[:, length:].any()
    with pytest.raises(ba.BonsaiAttnError):  # more rows than the target holds
        ba.kv_copy(ctx, ba.kv_state(d_kc, d_vc, 301), ba.kv_state(d_kc4, d_vc4, 0))


@pytest.mark.parametrize("n_layers,KV,cap_from,cap_to,length,shift", [
    (40, 1, 70, 33, 3, 0),        # 96 16-byte groups per layer: one partial chunk; 80 layer-caches in one grid
    (3, 4, 600, 520, 513, 0),     # 65,664 groups per layer: 64 whole chunks and a ragged 65th
    (2, 2, 300, 256, 256, 0),     # exactly 16 chunks per layer, target sized to the prefix
    (3, 2, 90, 80, 77, 4),        # caches 8 bytes off 16-byte alignment: the runtime's 2-D copies
])
def test_copy_ragged_and_unaligned(gpu, n_layers, KV, cap_from, cap_to, length, shift):
    torch, ctx, _ = gpu
    kc, vc = make_caches(0xE180 + length, n_layers, cap_from, KV, length)

    def placed(x):  # x on the device at `shift` int16 elements past an allocation's start
        flat = torch.zeros(x.size + shift, dtype=torch.int16, device="cuda")
        flat[shift:] = torch.from_numpy(np.ascontiguousarray(x).reshape(-1).view(np.int16)).cuda()
        return flat[shift:].view(x.shape)

    d_kc, d_vc = placed(kc), placed(vc)
    sentinel = np.full((n_layers, cap_to, KV, D), 0xFFFF, np.uint16)
    t_kc, t_vc = placed(sentinel), placed(sentinel)
    ba.kv_copy(ctx, ba.kv_state(d_kc, d_vc, length), ba.kv_state(t_kc, t_vc, 0))
    torch.cuda.synchronize()
    got_k, got_v = host16(t_kc), host16(t_vc)
    assert np.array_equal(got_k[:, :length], kc[:, :length]) and np.array_equal(got_v[:, :length], vc[:, :length])
    assert np.all(got_k[:, length:] == 0xFFFF) and np.all(got_v[:, length:] == 0xFFFF)


def test_attention_over_restored_cache_is_identical(gpu):
    torch, ctx, ws = gpu
    inp = workload.layer(0xE200, T=1, off=999, H=8, KV=2)  # cache rows 0..999 hold the prefix, row 999 is new
    n_layers = 2
    kc = np.stack([inp["kc"]] * n_layers)
    vc = np.stack([inp["vc"]] * n_layers)
    d_kc, d_vc = dev16(torch, kc), dev16(torch, vc)
    data = ba.kv_section_save(ctx, ba.kv_state(d_kc, d_vc, 999))
    r_kc = torch.zeros_like(d_kc)
    r_vc = torch.zeros_like(d_vc)
    ba.kv_section_load(ctx, data, ba.kv_state(r_kc, r_vc, 0))
    d = attn_to_dev(torch, inp)
    outs = []
    for ck, cv in ((d_kc[1], d_vc[1]), (r_kc[1], r_vc[1])):
        outs.append(ba.attention(ctx, ws, d["q"], ck, cv, 999, k_new=d["k_new"], v_new=d["v_new"],
                                 gate=d["gate"]).cpu().numpy())
    assert np.array_equal(outs[0], outs[1])


def test_bad_section_leaves_cache_untouched(gpu):
    torch, ctx, _ = gpu
    kc, vc = make_caches(0xE300, 2, 50, 1, 20)
    d_kc, d_vc = dev16(torch, kc), dev16(torch, vc)
    data = ba.kv_section_save(ctx, ba.kv_state(d_kc, d_vc, 20))
    target = torch.zeros_like(d_kc), torch.zeros_like(d_vc)
    for bad in (b"BNSPFX01" + data[8:], data[:-1], data[:12] + struct.pack("<I", 4 * D) + data[16:]):
        with pytest.raises(ba.BonsaiAttnError):
            ba.kv_section_load(ctx, bad, ba.kv_state(*target, 0))
    torch.cuda.synchronize()
    assert not host16(target[0]).any() and not host16(target[1]).any()
