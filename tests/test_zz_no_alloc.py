"""bn_attn_decode_ragged_noalloc (the ragged decode with its split partials in the library's per-device scratch
array instead of a caller workspace) against bn_attn_decode_ragged, through the C ABI on the GPU.

Both calls run the same kernels with the same split plan, so their outputs must be bit-identical; each is also held
to the oracle (max-abs 2e-3, projected argmax) and to bit-exact fp16 cache rows. Two noalloc calls run back to
back, the second with a smaller batch, so the second one runs over whatever the first left in the shared array.
"""
import numpy as np
import pytest

import oracle
from glimpse_language_amd import bonsai_attn as ba
from test_gpu_attn import assert_parity, cache_np, make_ragged

pytestmark = pytest.mark.gpu


def _batch(torch, seed, nseq, H, KV, lo, hi):
    lens, offs, kc, vc, q, k_new, v_new, z = make_ragged(seed, nseq, H, KV, lo, hi)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    for i in range(nseq):  # the new row of sequence i goes to its last row
        r = offs[i] + lens[i] - 1
        kc_ref[r] = k_new[i].astype(np.float16).view(np.uint16)
        vc_ref[r] = v_new[i].astype(np.float16).view(np.uint16)
    ref = oracle.decode_ragged(q, kc_ref, vc_ref, offs, lens, z)
    ref16 = oracle.decode_ragged(q, kc_ref, vc_ref, offs, lens, z, p16=True)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    dev = dict(q=t(q), offs=t(offs), lens=t(lens), k_new=t(k_new), v_new=t(v_new), z=t(z))
    return lens, kc, vc, kc_ref, vc_ref, (ref, ref16), dev


@pytest.mark.parametrize("first,second", [
    ((0x7A11, 32, 16, 4, 1024, 8192), (0x7A12, 5, 8, 2, 100, 3000)),
])
def test_noalloc_matches_workspace_call(gpu, first, second):
    torch, ctx, ws = gpu
    for seed, nseq, H, KV, lo, hi in (first, second):
        print(f"noalloc ragged decode: seed {seed:#x}, {nseq} sequences, {H}q/{KV}kv, L in [{lo}, {hi}]", flush=True)
        lens, kc, vc, kc_ref, vc_ref, ref, d = _batch(torch, seed, nseq, H, KV, lo, hi)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
        kc_a, vc_a = t(kc.view(np.int16)), t(vc.view(np.int16))
        kc_b, vc_b = t(kc.view(np.int16)), t(vc.view(np.int16))
        max_len = int(lens.max())
        out_ws = ba.decode_ragged(ctx, ws, d["q"], kc_a, vc_a, d["offs"], d["lens"], max_len, k_new=d["k_new"],
                                  v_new=d["v_new"], gate=d["z"])
        out_na = ba.decode_ragged_noalloc(ctx, d["q"], kc_b, vc_b, d["offs"], d["lens"], max_len, k_new=d["k_new"],
                                          v_new=d["v_new"], gate=d["z"])
        torch.cuda.synchronize()
        a, b = out_ws.cpu().numpy(), out_na.cpu().numpy()
        assert np.array_equal(a, b), f"noalloc differs from the workspace call by {np.max(np.abs(a - b)):.3e}"
        assert_parity(b, ref[0], H, "noalloc", ref[1])
        assert np.array_equal(cache_np(kc_b), kc_ref) and np.array_equal(cache_np(vc_b), vc_ref)
        assert np.array_equal(cache_np(kc_a), kc_ref) and np.array_equal(cache_np(vc_a), vc_ref)


def test_noalloc_rejects_a_batch_beyond_the_scratch_array(gpu):
    """A batch whose partials exceed the array is refused before any launch (outputs untouched)."""
    torch, ctx, _ = gpu
    nseq, H, KV = 4000, 16, 4
    q = torch.zeros(nseq, H, 256, device="cuda")
    kc = torch.zeros(nseq, KV, 256, dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    offs = torch.arange(nseq, dtype=torch.int64, device="cuda")
    lens = torch.ones(nseq, dtype=torch.int32, device="cuda")
    out = torch.full((nseq, H, 256), 7.0, device="cuda")
    with pytest.raises(ba.BonsaiAttnError) as e:
        ba.decode_ragged_noalloc(ctx, q, kc, vc, offs, lens, 100000, out=out)
    assert e.value.status == ba.BN_ENOWS
    assert "scratch" in ctx.error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
