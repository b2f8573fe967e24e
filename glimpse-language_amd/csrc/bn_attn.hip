// C ABI of the gfx950 attention path (include/bonsai_attn.h): argument checks, split policy, workspace
// layout and kernel launches. Host logic only; the kernels live in the bn_*.h headers.
#include "bonsai_attn.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <tuple>
#include <utility>

#include "bn_decode.h"
#include "bn_flash.h"
#include "bn_prefill.h"
#include "bn_prefill_hilo.h"
#include "bn_prefill_pair.h"
#include "bn_prep.h"
#include "bn_ternary.h"
#include "bn_ternary_pf.h"
#include "bn_util_kernels.h"
#include "bn_verify.h"

struct bn_ctx {
    int device;
    int cus;
    // T >= 2 calls use prefill_kernel when they give at least this many 32-token q-tile blocks (default: the
    // CU count; BONSAI_ATTN_PREFILL_MIN_BLOCKS overrides it at context creation, e.g. 1 in tests)
    int prefill_min_blocks;
    // waves per decode split block (1, 2, 4 or 8; BONSAI_ATTN_DECODE_WAVES overrides it at context creation; 16 waves
    // left the kernel 128 registers per lane and spilled, so it is not offered)
    int decode_waves;
    // waves a decode launch aims at (256 .. BN_DECODE_MAX_TARGET_WAVES; BONSAI_ATTN_DECODE_TARGET_WAVES)
    int decode_target_waves;
    // splits of one sequence at most (1 .. kMaxSplitsCap; BONSAI_ATTN_DECODE_MAX_SPLITS)
    int decode_max_splits;
    // blocks flash_kernel's key splits aim at (1 .. kFlashTargetBlocks; BONSAI_ATTN_FLASH_TARGET_BLOCKS)
    int flash_target_blocks;
    // 2..16 verify rows on verify_kernel (1, the default) or as decodes of their rows (0; BONSAI_ATTN_VERIFY_MFMA)
    int verify_mfma;
    // fp16-q prefills on prefill_kernel (0, the default) or prefill_pair_kernel (1; BONSAI_ATTN_PREFILL_PAIR=1)
    int prefill_pair;
    // 17..64 rows too few for prefill_kernel: verify_kernel's row groups (1, the default) or flash_kernel (0;
    // BONSAI_ATTN_MID_ROWS)
    int mid_rows;
    // this device's copy of `scratch` (the partials of bn_attn_decode_ragged_noalloc), or null if its address
    // could not be taken
    void* scratch;
    // the first failed launch since the last status check (bn_launch's own return value), or hipSuccess
    hipError_t launch_err;
    char err[256];
};

// Split partials of bn_attn_decode_ragged_noalloc, for callers that cannot allocate. The code object holds one
// copy per device from its load until the process ends. Host code uses the array only through the per-device
// address that hipGetSymbolAddress gives (scratch_address); its name is not a device address on the host.
// BN_NOALLOC_SCRATCH_BYTES (16 MiB) is in the header.
static __device__ __align__(256) float scratch[BN_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

thread_local char g_check_err[256];

constexpr int kVerifyMax = 16;     // verify rows handled by the verify kernel (model.rs VMAX = 16)
constexpr int64_t kMaxRows = 1 << 24;  // positions addressable by one call (int32 key indices)

bn_status set_err(char* buf, bn_status s, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, 256, fmt, ap);
    va_end(ap);
    return s;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int64_t ceil_div(int64_t x, int64_t m) { return (x + m - 1) / m; }

#ifndef BN_DECODE_TARGET_WAVES
#define BN_DECODE_TARGET_WAVES 2048
#endif
// the workspace query sizes the partials for this many waves (the largest target a context may use)
#define BN_DECODE_MAX_TARGET_WAVES 4096
#ifndef BN_DECODE_WAVES
#define BN_DECODE_WAVES 2
#endif
#ifndef BN_DECODE_MAX_SPLITS
#define BN_DECODE_MAX_SPLITS 64
#endif
// the workspace query sizes the partials without a cap on the splits of one sequence
constexpr int64_t kMaxSplitsCap = 1 << 20;

// Single-token decodes: about `target_waves` waves over the launch in blocks of W waves, i.e.
// target = target_waves / (W KV) units per kv head. In flat order (bn_decode.h) a unit is an equal run of the
// batch's concatenated keys (the kernels derive the chunk from the device-side lengths with bn::dec_chunk_flat), so
// the launch is at most `target` units wide per kv head whatever the lengths (a batch of sequences cut per sequence
// left up to nseq more, partly filled blocks: 1088 blocks against 1024 resident slots for 32 ragged sequences).
// No sequence spans more than max_splits + 1 units (the merge of one sequence runs on two blocks per kv head, so a long
// single sequence cut into hundreds of splits would wait on its merge: 95 us against 27 us for 16K keys with the cap
// at 64). Records: segment (unit b, sequence i) in slot b + i, so units + nseq slots. The workspace query has no
// context, so it sizes the partials for W = 1 and BN_DECODE_MAX_TARGET_WAVES, the most units a context gives.
struct DecodePlan {
    int64_t nseq, KV, max_len, target, max_splits, units, slots, waves;
    bool multi;  // some sequence may take more than one unit (then the partials need the workspace)
    bool xcd_rows = false;  // rows of one sequence in the XCD-aware unit order (bn::DecodeArgs::xcd_rows)
    size_t part_bytes;
    size_t total() const { return multi ? part_bytes : 0; }
};

DecodePlan plan_decode(int64_t nseq, int64_t KV, int64_t max_len, int64_t known_len, int64_t waves,
                       int64_t target_waves, int64_t max_splits) {
    DecodePlan p;
    p.nseq = nseq;
    p.KV = KV;
    p.max_len = max_len;
    p.waves = waves;
    p.target = target_waves / (waves * KV);
    if (p.target < 1) p.target = 1;
    p.max_splits = max_splits;
    if (known_len >= 0) {
        // one sequence of known length: the exact unit count
        const int64_t chunk = bn::dec_chunk_flat(known_len, (int)p.target, (int)max_len, (int)p.max_splits);
        p.units = known_len > 0 ? ceil_div(known_len, chunk) : 1;
        p.slots = p.units;
        p.multi = p.units > 1;
    } else {
        // ceil(sum L / chunk) <= target units, and chunk >= 64
        p.units = p.target;
        const int64_t by_len = ceil_div(nseq * max_len, bn::DEC_MIN_CHUNK);
        if (by_len < p.units) p.units = by_len;
        p.slots = p.units + nseq;
        p.multi = nseq * max_len > bn::DEC_MIN_CHUNK;
    }
    p.part_bytes = (size_t)(KV * p.slots) * bn::DEC_PART * sizeof(float);
    return p;
}

// T query rows of one sequence run as T single-token decodes: row t attends to off + t + 1 keys (causal among the
// rows). The lengths are known on the host, so the split count is exact; with a device offset (a->dyn) `off` is
// only their upper bound, and the launch covers every split count the kernels can derive from a smaller offset.
DecodePlan plan_rows(const bn_attn_args* a, int64_t waves, int64_t target_waves, int64_t max_splits) {
    const int64_t T = a->T, off = a->off;
    const bool exact = a->dyn == nullptr;
    DecodePlan p = plan_decode(T, a->KV, off + T, (T == 1 && exact) ? off + 1 : -1, waves, target_waves, max_splits);
    if (T > 1 && !exact) {
        // For any device offset d <= off the kernels' chunk is at least 64 keys, (off + T) / max_splits keys and
        // sum / target keys, sum = T (d + 1) + T (T - 1) / 2 >= T (L - T + 1) the rows' keys (L = d + T, the longest
        // row), so a row takes at most L target / (T (L - T + 1)) + 1 splits: at most 2 target / T + 1 when
        // L >= 2T - 1, and at most ceil((2T - 2) / 64) by the 64-key floor below that.
        int64_t ns_max = ceil_div(off + T, bn::DEC_MIN_CHUNK);
        if (ns_max > max_splits) ns_max = max_splits;
        int64_t by_target = 2 * p.target / T + 1;
        const int64_t short_rows = ceil_div(2 * T - 2, bn::DEC_MIN_CHUNK);
        if (by_target < short_rows) by_target = short_rows;
        if (ns_max > by_target) ns_max = by_target;
        p.xcd_rows = true;
        p.units = 8 * T * ceil_div(ns_max, 8);
        p.slots = p.units;
        p.multi = ns_max > 1;
        p.part_bytes = (size_t)(a->KV * p.units) * bn::DEC_PART * sizeof(float);
    } else if (T > 1) {
        // every row reads the same cache rows: split s of all rows goes to one XCD (units 8 (t + T (s / 8)) +
        // s % 8), so each split's K/V rows come from HBM once and from that XCD's L2 for the other rows
        const int64_t sum = T * (off + 1) + T * (T - 1) / 2;
        const int64_t chunk = bn::dec_chunk(sum, (int)p.target, (int)(off + T), (int)p.max_splits);
        const int64_t ns_max = ceil_div(off + T, chunk);
        p.xcd_rows = true;
        p.units = 8 * T * ceil_div(ns_max, 8);
        p.slots = p.units;
        p.multi = ns_max > 1;
        p.part_bytes = (size_t)(a->KV * p.units) * bn::DEC_PART * sizeof(float);
    }
    return p;
}

// T >= 2 rows: q-tiles of 32 tokens; the key range of a q-tile is split only when the q-tiles alone give
// fewer blocks than CUs (then about 512 blocks of equal key tiles). Depends only on the shapes.
// flash_kernel's key splits aim at about this many blocks (the workspace query sizes the partials for it; a context
// may aim lower: BONSAI_ATTN_FLASH_TARGET_BLOCKS)
constexpr int64_t kFlashTargetBlocks = 512;

struct FlashPlan {
    int64_t ntq, ct, max_splits;
    size_t acc_bytes, ml_bytes;
    size_t total() const { return max_splits > 1 ? acc_bytes + ml_bytes : 0; }
};

FlashPlan plan_flash(int64_t T, int64_t off, int64_t KV, int64_t target_blocks = kFlashTargetBlocks) {
    FlashPlan p;
    p.ntq = ceil_div(T, bn::FL_BQ);
    const int64_t max_kt = ceil_div(off + T, bn::FL_BK);
    if (KV * p.ntq >= 256) {
        p.ct = max_kt;
    } else {
        int64_t iters = 0;
        for (int64_t qt = 0; qt < p.ntq; qt++) {
            const int64_t t_last = (qt + 1) * bn::FL_BQ < T ? (qt + 1) * bn::FL_BQ : T;
            iters += ceil_div(off + t_last, bn::FL_BK);
        }
        iters *= KV;
        p.ct = ceil_div(iters, target_blocks);
        if (p.ct < 1) p.ct = 1;
    }
    p.max_splits = ceil_div(max_kt, p.ct);
    const int64_t rows = KV * p.ntq * p.max_splits * bn::FL_ROWS;
    p.acc_bytes = (size_t)rows * bn::D * sizeof(float);
    p.ml_bytes = (size_t)rows * 2 * sizeof(float);
    return p;
}

// T >= 2 rows with enough 32-token q-tiles to fill the GPU: prefill_kernel (one block per q-tile, the key range
// split between the block's two wave groups). Depends only on the shapes and the context's threshold.
bool use_prefill(const bn_attn_args* a, int64_t min_blocks) {
    return a->T >= 2 && (int64_t)a->KV * ceil_div(a->T, bn::PF_BQ) >= min_blocks;
}

// The LoRA-A rows of a call: A [r][k] fp16 (16-byte aligned, k staged in LDS), u rows of at least r floats.
bn_status check_lora(const uint16_t* A, const float* U, int64_t u_ts, uint32_t r, int64_t T, int64_t k, int64_t k_max,
                     char* why) {
    if (!r) return BN_OK;
    if (r > 4096) return set_err(why, BN_EINVAL, "lora_r must be at most 4096 (lora_r=%u)", r);
    if (!A || !U || !aligned16(A) || ((uintptr_t)U & 3))
        return set_err(why, BN_EINVAL, "lora_a (16-byte aligned) and lora_u are required with lora_r");
    if (k > k_max) return set_err(why, BN_EINVAL, "LoRA rows over %lld columns, at most %lld", (long long)k, (long long)k_max);
    if (u_ts < 0 || (T > 1 && u_ts < (int64_t)r)) return set_err(why, BN_EINVAL, "lora_us must be at least lora_r");
    return BN_OK;
}

bn_status check_attn(const bn_attn_args* a, int kind, char* why) {
    if (!a) return set_err(why, BN_EINVAL, "args is NULL");
    if (kind < 0 || kind > 4) return set_err(why, BN_EINVAL, "unknown kind %d", kind);
    if (a->KV < 1 || a->H != 4 * a->KV)
        return set_err(why, BN_EINVAL, "need H == 4*KV >= 4 (H=%u KV=%u)", a->H, a->KV);
    if (a->T < 1) return set_err(why, BN_EINVAL, "T must be >= 1");
    if (kind == 1 && a->T != 1) return set_err(why, BN_EINVAL, "decode takes T == 1 (T=%u)", a->T);
    if (kind == 2 && a->T > (uint32_t)kVerifyMax)
        return set_err(why, BN_EINVAL, "verify takes T <= %d (T=%u)", kVerifyMax, a->T);
    if ((uint64_t)a->off + a->T > a->cap)
        return set_err(why, BN_EINVAL, "off + T = %llu exceeds cap = %u", (unsigned long long)a->off + a->T, a->cap);
    if ((int64_t)a->off + a->T > kMaxRows) return set_err(why, BN_EINVAL, "off + T beyond %lld", (long long)kMaxRows);
    if (a->flags & ~BN_Q_F16) return set_err(why, BN_EINVAL, "unknown flags 0x%x", a->flags);
    if (!a->kc || !a->vc) return set_err(why, BN_EINVAL, "kc and vc are required");
    if (!aligned16(a->kc) || !aligned16(a->vc)) return set_err(why, BN_EINVAL, "kc/vc must be 16-byte aligned");
    if ((a->k_new == nullptr) != (a->v_new == nullptr))
        return set_err(why, BN_EINVAL, "k_new and v_new are given together or not at all");
    if (a->k_new && (!aligned16(a->k_new) || !aligned16(a->v_new)))
        return set_err(why, BN_EINVAL, "k_new/v_new must be 16-byte aligned");
    if (kind == 4) {
        if (!a->k_new) return set_err(why, BN_EINVAL, "append needs k_new and v_new");
        return BN_OK;
    }
    if (!a->q || !a->out) return set_err(why, BN_EINVAL, "q and out are required");
    if (!aligned16(a->out) || (a->o_ts & 3) || (a->o_hs & 3) || a->o_ts < 0 || a->o_hs < 0)
        return set_err(why, BN_EINVAL, "out must be 16-byte aligned with strides that are multiples of 4 floats");
    const int64_t qv = (a->flags & BN_Q_F16) ? 8 : 4;  // elements per 16 bytes
    if (a->q_ts < 0 || a->q_hs < 0 || !aligned16(a->q) || (a->q_ts % qv) || (a->q_hs % qv))
        return set_err(why, BN_EINVAL, "q must be 16-byte aligned with strides that are whole 16-byte groups");
    // the kernels read the gate 16 bytes at a time
    if (a->gate && (a->g_ts < 0 || a->g_hs < 0 || !aligned16(a->gate) || (a->g_ts & 3) || (a->g_hs & 3)))
        return set_err(why, BN_EINVAL, "gate must be 16-byte aligned with strides that are multiples of 4 floats");
    if (a->signs && !aligned16(a->signs)) return set_err(why, BN_EINVAL, "signs must be 16-byte aligned");
    bn_status ls = check_lora(a->lora_a, a->lora_u, a->lora_us, a->lora_r, a->T, (int64_t)a->H * bn::D, bn::LORA_MAX_K, why);
    if (ls) return ls;
    size_t need = bn_attn_workspace_size(a);
    if (need && (!a->ws || a->ws_bytes < need || !aligned16(a->ws)))
        return set_err(why, BN_ENOWS, "workspace needs %zu bytes (16-byte aligned), got %zu", need, a->ws_bytes);
    return BN_OK;
}

bn_status check_ragged(const bn_ragged_args* a, char* why, bool own_ws = true) {
    if (!a) return set_err(why, BN_EINVAL, "args is NULL");
    if (a->nseq < 1 || a->nseq > 65535) return set_err(why, BN_EINVAL, "nseq must be in 1..65535");
    if (a->KV < 1 || a->H != 4 * a->KV)
        return set_err(why, BN_EINVAL, "need H == 4*KV >= 4 (H=%u KV=%u)", a->H, a->KV);
    if (a->max_len < 1 || a->max_len > kMaxRows) return set_err(why, BN_EINVAL, "max_len out of range");
    if (!a->q || !a->out || !a->kc || !a->vc || !a->kv_off || !a->kv_len)
        return set_err(why, BN_EINVAL, "q, out, kc, vc, kv_off and kv_len are required");
    if (!aligned16(a->kc) || !aligned16(a->vc)) return set_err(why, BN_EINVAL, "kc/vc must be 16-byte aligned");
    if ((a->k_new == nullptr) != (a->v_new == nullptr))
        return set_err(why, BN_EINVAL, "k_new and v_new are given together or not at all");
    if (a->k_new && (!aligned16(a->k_new) || !aligned16(a->v_new)))
        return set_err(why, BN_EINVAL, "k_new/v_new must be 16-byte aligned");
    if (!aligned16(a->out) || (a->o_ss & 3) || (a->o_hs & 3) || a->o_ss < 0 || a->o_hs < 0)
        return set_err(why, BN_EINVAL, "out must be 16-byte aligned with strides that are multiples of 4 floats");
    // q and the gate are read 16 bytes at a time
    if (a->q_ss < 0 || a->q_hs < 0 || !aligned16(a->q) || (a->q_ss & 3) || (a->q_hs & 3))
        return set_err(why, BN_EINVAL, "q must be 16-byte aligned with strides that are multiples of 4 floats");
    if (a->gate && (a->g_ss < 0 || a->g_hs < 0 || !aligned16(a->gate) || (a->g_ss & 3) || (a->g_hs & 3)))
        return set_err(why, BN_EINVAL, "gate must be 16-byte aligned with strides that are multiples of 4 floats");
    if (a->signs && !aligned16(a->signs)) return set_err(why, BN_EINVAL, "signs must be 16-byte aligned");
    if (!own_ws) return BN_OK;
    size_t need = bn_ragged_workspace_size(a);
    if (need && (!a->ws || a->ws_bytes < need || !aligned16(a->ws)))
        return set_err(why, BN_ENOWS, "workspace needs %zu bytes (16-byte aligned), got %zu", need, a->ws_bytes);
    return BN_OK;
}

bn_status check_prep(const bn_prep_args* a, char* why, bool q_optional = false) {
    if (!a) return set_err(why, BN_EINVAL, "args is NULL");
    if (a->KV < 1 || a->H != 4 * a->KV)
        return set_err(why, BN_EINVAL, "need H == 4*KV >= 4 (H=%u KV=%u)", a->H, a->KV);
    if (a->T < 1) return set_err(why, BN_EINVAL, "T must be >= 1");
    if ((uint64_t)a->off + a->T > a->cap)
        return set_err(why, BN_EINVAL, "off + T = %llu exceeds cap = %u", (unsigned long long)a->off + a->T, a->cap);
    if ((int64_t)a->off + a->T > kMaxRows) return set_err(why, BN_EINVAL, "off + T beyond %lld", (long long)kMaxRows);
    if (a->flags & ~BN_Q_F16) return set_err(why, BN_EINVAL, "unknown flags 0x%x", a->flags);
    if ((a->rot & 7) || a->rot > (uint32_t)bn::D)
        return set_err(why, BN_EINVAL, "rot must be a multiple of 8 in 0..256 (rot=%u)", a->rot);
    if (!a->qp || !a->kp || !a->vp || !a->q_norm || !a->k_norm || (!a->q && !q_optional) || !a->kc || !a->vc)
        return set_err(why, BN_EINVAL, "qp, kp, vp, q_norm, k_norm, q, kc and vc are required");
    if (a->rot && (!a->pos || !a->inv_freq)) return set_err(why, BN_EINVAL, "pos and inv_freq are required when rot > 0");
    if (!aligned16(a->qp) || !aligned16(a->kp) || !aligned16(a->vp) || !aligned16(a->q_norm) ||
        !aligned16(a->k_norm) || !aligned16(a->q) || !aligned16(a->kc) || !aligned16(a->vc))
        return set_err(why, BN_EINVAL, "qp, kp, vp, q_norm, k_norm, q, kc and vc must be 16-byte aligned");
    if (a->qp_ts < 0 || a->qp_hs < 0 || (a->qp_ts & 3) || (a->qp_hs & 3) || a->q_ts < 0 || a->q_hs < 0 ||
        (a->q_ts & 3) || (a->q_hs & 3))
        return set_err(why, BN_EINVAL, "qp and q strides must be non-negative multiples of 4 elements");
    if ((const void*)a->qp == a->q && ((a->flags & BN_Q_F16) || a->qp_ts != a->q_ts || a->qp_hs != a->q_hs))
        return set_err(why, BN_EINVAL, "q may be qp itself only in fp32 with the same strides");
    return BN_OK;
}

bn_status check_rotate(const bn_rotate_args* a, char* why) {
    if (!a) return set_err(why, BN_EINVAL, "args is NULL");
    if (a->T < 1 || a->T > (1u << 30)) return set_err(why, BN_EINVAL, "T must be in 1..2^30");
    if (a->H < 2 || (a->H & 1) || a->H > 2u * 65535u)
        return set_err(why, BN_EINVAL, "H must be even, 2..131070 (H=%u)", a->H);
    if (!a->attn || !a->signs || !a->xr) return set_err(why, BN_EINVAL, "attn, signs and xr are required");
    if (!aligned16(a->attn) || !aligned16(a->signs) || !aligned16(a->xr) || !aligned16(a->gate))
        return set_err(why, BN_EINVAL, "attn, gate, signs and xr must be 16-byte aligned");
    if (a->a_ts < 0 || a->x_ts < 0 || (a->a_ts & 3) || (a->x_ts & 3) ||
        (a->gate && (a->g_ts < 0 || a->g_hs < 0 || (a->g_ts & 3) || (a->g_hs & 3))))
        return set_err(why, BN_EINVAL, "strides must be non-negative multiples of 4 elements");
    if ((const float*)a->xr == a->attn && a->x_ts != a->a_ts)
        return set_err(why, BN_EINVAL, "xr may be attn itself only with the same stride");
    if (a->lora_r && (const float*)a->xr == a->attn)
        return set_err(why, BN_EINVAL, "with LoRA rows xr may not be attn (they read the gated rows)");
    return check_lora(a->lora_a, a->lora_u, a->lora_us, a->lora_r, a->T, (int64_t)a->H * bn::D, bn::LORA_MAX_K, why);
}

// The device address of `scratch` on `device`, taken once per device with that device current (each GPU holds
// its own copy at its own address) and kept for the life of the process; null if the runtime refuses.
void* scratch_address(int device) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* addr[kMaxDevices];
    static bool tried[kMaxDevices];
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!tried[device]) {
        tried[device] = true;
        int prev = -1;
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        void* p = nullptr;
        if (hipSetDevice(device) == hipSuccess && hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess)
            addr[device] = p;
        if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    }
    return addr[device];
}

// Kernels are launched with hipLaunchKernel, whose return value is that launch's own status: the <<<>>> form
// returns nothing, and the thread's sticky last error it leaves behind may also hold an error of other code on
// the thread (which reading it would clear). The first failure since the last check is kept in the context.
template <typename K, typename Vals, size_t... I>
hipError_t launch_vals(K* kern, dim3 grid, dim3 block, size_t shm, hipStream_t st, Vals& vals,
                       std::index_sequence<I...>) {
    void* ptrs[] = {static_cast<void*>(&std::get<I>(vals))...};
    return hipLaunchKernel(reinterpret_cast<const void*>(kern), grid, block, ptrs, shm, st);
}
template <typename... P, typename... A>
void bn_launch(bn_ctx* ctx, void (*kern)(P...), dim3 grid, dim3 block, size_t shm, hipStream_t st, A&&... args) {
    static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
    std::tuple<P...> vals(static_cast<P>(args)...);
    const hipError_t e = launch_vals(kern, grid, block, shm, st, vals, std::index_sequence_for<P...>{});
    if (e != hipSuccess && ctx->launch_err == hipSuccess) ctx->launch_err = e;
}

bn_status launched(bn_ctx* ctx, const char* what) {
    const hipError_t e = ctx->launch_err;
    ctx->launch_err = hipSuccess;
    if (e != hipSuccess) return set_err(ctx->err, BN_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
    return BN_OK;
}

bn_status launch_append(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a) {
    const int64_t row = (int64_t)a->KV * bn::D;
    const int64_t n8 = (int64_t)a->T * row / 8;
    int64_t blocks = ceil_div(n8, 256);
    if (blocks > 4096) blocks = 4096;
    bn_launch(ctx, bn::append_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a->k_new, a->v_new, a->kc, a->vc,
                       row, (int)a->off, a->dyn, n8);
    return launched(ctx, "append_kernel");
}

bn_status launch_decode(bn_ctx* ctx, hipStream_t st, const bn::DecodeArgs& d, const DecodePlan& p) {
    const dim3 grid((unsigned)p.units, (unsigned)p.KV);
    switch (p.waves) {
        case 1: bn_launch(ctx, bn::decode_split_kernel<1>, grid, dim3(64), 0, st, d); break;
        case 2:
            // cached K/V loads where rows are shared (xcd_rows) or the launch holds at most one block per CU
            // (latency-bound: single-sequence decodes over 32K keys 0.3-1 us faster, the rest unchanged); the wide
            // streaming launches keep non-temporal loads (32 x 8K keys: 173-174 against 190-194 us cached)
            if (p.xcd_rows || p.units * p.KV <= (int64_t)ctx->cus)
                bn_launch(ctx, (bn::decode_split_kernel<2, true>), grid, dim3(128), 0, st, d);
            else
                bn_launch(ctx, (bn::decode_split_kernel<2, false>), grid, dim3(128), 0, st, d);
            break;
        case 4: bn_launch(ctx, bn::decode_split_kernel<4>, grid, dim3(256), 0, st, d); break;
        default: bn_launch(ctx, bn::decode_split_kernel<8>, grid, dim3(512), 0, st, d); break;
    }
    bn_status s = launched(ctx, "decode_split_kernel");
    if (s || !p.multi) return s;
    bn_launch(ctx, bn::decode_combine_kernel, dim3((unsigned)p.nseq, (unsigned)(2 * p.KV)), dim3(512), 0, st, d);
    return launched(ctx, "decode_combine_kernel");
}

void bind_workspace(bn::DecodeArgs& d, const DecodePlan& p, void* ws) {
    d.nseq = (int)p.nseq;
    d.max_len = (int)p.max_len;
    d.target = (int)p.target;
    d.max_splits = (int)p.max_splits;
    d.units = (int)p.slots;
    d.xcd_rows = p.xcd_rows;
    d.part = p.multi ? static_cast<float*>(ws) : nullptr;
}

// Query rows as single-token decodes (row t over off + t + 1 keys, the sequence's rows at stride q_ts). One row
// fuses its append into the split kernel (the new row is its last key); several rows append first, since row t
// reads the new rows before it from the cache.
// rp (optional): attn_prep in the kernels' prologue; a->q and, for one row, a->k_new are then raw q_proj / k_proj
// rows (several rows have their K/V rows written by prep_kernel before this call).
bn_status run_rows(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a, const bn::RopeParams* rp = nullptr) {
    DecodePlan p = plan_rows(a, ctx->decode_waves, ctx->decode_target_waves, ctx->decode_max_splits);
    const bool fused = a->T == 1;
    if (!fused && a->k_new) {
        bn_status s = launch_append(ctx, st, a);
        if (s) return s;
    }
    bn::DecodeArgs d{};
    if (a->flags & BN_Q_F16)
        d.q16 = static_cast<const uint16_t*>(a->q);
    else
        d.q = static_cast<const float*>(a->q);
    d.q_ss = a->q_ts;
    d.q_hs = a->q_hs;
    d.k_new = fused ? a->k_new : nullptr;
    d.v_new = fused ? a->v_new : nullptr;
    d.kn_ss = (int64_t)a->KV * bn::D;
    d.kc = a->kc;
    d.vc = a->vc;
    d.row0 = 0;
    d.row_step = 0;
    d.len0 = (int32_t)a->off + 1;
    d.len_step = 1;
    d.dyn = a->dyn;
    d.gate = a->gate;
    d.g_ss = a->g_ts;
    d.g_hs = a->g_hs;
    d.out = a->out;
    d.o_ss = a->o_ts;
    d.o_hs = a->o_hs;
    d.signs = a->signs;
    if (rp) d.rp = *rp;
    d.KV = (int)a->KV;
    bind_workspace(d, p, a->ws);
    return launch_decode(ctx, st, d, p);
}

#ifndef BN_VERIFY_WAVES
#define BN_VERIFY_WAVES 4
#endif
#ifndef BN_VERIFY_BLOCKS
#define BN_VERIFY_BLOCKS 128
#endif
constexpr int kVerifyMfmaMax = 16;  // two row groups of 8 (4 heads x 8 rows: one 32-column MFMA tile each)

// verify_kernel's keys per split for 2..16 rows: about BN_VERIFY_BLOCKS blocks over the kv heads, whole 32-key tiles
// for each of the W waves, and never more splits than the workspace query sized (its chunk is a lower bound).
// 0 when the workspace holds no partials (a short context: every row fits one split of the decode path).
int64_t verify_chunk(const bn_attn_args* a) {
    if (a->T < 2 || a->T > (uint32_t)kVerifyMfmaMax) return 0;
    const int64_t T = a->T, off = a->off, nk = off + T;
    const DecodePlan ws = plan_rows(a, 1, BN_DECODE_MAX_TARGET_WAVES, kMaxSplitsCap);
    if (!ws.multi) return 0;
    const int64_t sum = T * (off + 1) + T * (T - 1) / 2;
    const int64_t ws_chunk = bn::dec_chunk(sum, (int)ws.target, (int)nk, (int)ws.max_splits);
    const int64_t step = 32 * BN_VERIFY_WAVES;
    int64_t c = ceil_div(nk * a->KV, BN_VERIFY_BLOCKS);
    if (c < ws_chunk) c = ws_chunk;
    return ceil_div(c, step) * step;
}

// bn_attn_layer's fp32 q rows for verify_kernel when the caller gives no q output: after the partials in the
// workspace (256-byte aligned), T x H x 256 fp32
size_t verify_q_offset(const bn_attn_args* a) {
    return (plan_rows(a, 1, BN_DECODE_MAX_TARGET_WAVES, kMaxSplitsCap).total() + 255) / 256 * 256;
}

// 2..16 rows of one sequence on verify_kernel (every K/V row read once per group of 8 rows), then
// decode_combine_kernel for the merge, the gate and the rotation. The rows' K/V, when given, are appended by
// verify_kernel itself.
bn_status run_verify(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a, int64_t chunk) {
    const int64_t T = a->T, nk = (int64_t)a->off + T, ns = ceil_div(nk, chunk);
    const unsigned groups = (unsigned)ceil_div(T, 8);
    const int64_t units = 8 * T * ceil_div(ns, 8);
    bn::VerifyArgs v{};
    if (a->flags & BN_Q_F16)
        v.q16 = static_cast<const uint16_t*>(a->q);
    else
        v.q = static_cast<const float*>(a->q);
    v.q_ts = a->q_ts;
    v.q_hs = a->q_hs;
    v.kc = a->kc;
    v.vc = a->vc;
    v.k_new = a->k_new;  // appended by the kernel (the wave that owns each new row's tile)
    v.v_new = a->v_new;
    v.part = static_cast<float*>(a->ws);
    v.dyn = a->dyn;
    v.T = (int)T;
    v.off = (int)a->off;
    v.KV = (int)a->KV;
    v.chunk = (int)chunk;
    v.units = (int)units;
    if (v.q)
        bn_launch(ctx, (bn::verify_kernel<BN_VERIFY_WAVES, true>), dim3((unsigned)ns, (unsigned)a->KV, groups),
                  dim3(64 * BN_VERIFY_WAVES), 0, st, v);
    else
        bn_launch(ctx, (bn::verify_kernel<BN_VERIFY_WAVES, false>), dim3((unsigned)ns, (unsigned)a->KV, groups),
                  dim3(64 * BN_VERIFY_WAVES), 0, st, v);
    bn_status s = launched(ctx, "verify_kernel");
    if (s) return s;
    bn::DecodeArgs d{};
    d.kc = a->kc;
    d.vc = a->vc;
    d.len0 = (int32_t)a->off + 1;
    d.len_step = 1;
    d.dyn = a->dyn;
    d.gate = a->gate;
    d.g_ss = a->g_ts;
    d.g_hs = a->g_hs;
    d.out = a->out;
    d.o_ss = a->o_ts;
    d.o_hs = a->o_hs;
    d.signs = a->signs;
    d.KV = (int)a->KV;
    d.nseq = (int)T;
    d.max_len = (int)nk;
    d.target = 1;
    d.max_splits = (int)ns;
    d.units = (int)units;
    d.xcd_rows = 1;
    d.chunk = (int)chunk;
    d.part = v.part;
    bn_launch(ctx, bn::decode_combine_kernel, dim3((unsigned)T, (unsigned)(2 * a->KV)), dim3(512), 0, st, d);
    return launched(ctx, "decode_combine_kernel");
}

bn_status run_prefill(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a) {
    bn::PrefillArgs f{};
    if (a->flags & BN_Q_F16)
        f.q16 = static_cast<const uint16_t*>(a->q);
    else
        f.q = static_cast<const float*>(a->q);
    f.q_ts = a->q_ts;
    f.q_hs = a->q_hs;
    f.kc = a->kc;
    f.vc = a->vc;
    f.gate = a->gate;
    f.g_ts = a->g_ts;
    f.g_hs = a->g_hs;
    f.out = a->out;
    f.o_ts = a->o_ts;
    f.o_hs = a->o_hs;
    f.signs = a->signs;
    f.dyn = a->dyn;
    f.T = (int)a->T;
    f.off = (int)a->off;
    f.KV = (int)a->KV;
    f.ntq = (int)ceil_div(a->T, bn::PF_BQ);
    const int64_t blocks = (int64_t)a->KV * f.ntq;
    if (f.q16 && ctx->prefill_pair) {
        bn_launch(ctx, bn::prefill_pair_kernel, dim3((unsigned)blocks), dim3(256), 0, st, f);
        return launched(ctx, "prefill_pair_kernel");
    }
    if (f.q16) {
        bn_launch(ctx, bn::prefill_kernel, dim3((unsigned)blocks), dim3(512), 0, st, f);
        return launched(ctx, "prefill_kernel");
    }
    bn_launch(ctx, bn::prefill_hilo_kernel, dim3((unsigned)blocks), dim3(256), 0, st, f);
    return launched(ctx, "prefill_hilo_kernel");
}

// T >= 2 rows: append, then the MFMA kernel (and the split merge when the key range is split).
bn_status attend_flash(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a) {
    if (a->k_new) {
        bn_status s = launch_append(ctx, st, a);
        if (s) return s;
    }
    if (use_prefill(a, ctx->prefill_min_blocks)) return run_prefill(ctx, st, a);
    FlashPlan p = plan_flash(a->T, a->off, a->KV, ctx->flash_target_blocks);
    bn::FlashArgs f{};
    if (a->flags & BN_Q_F16)
        f.q16 = static_cast<const uint16_t*>(a->q);
    else
        f.q = static_cast<const float*>(a->q);
    f.q_ts = a->q_ts;
    f.q_hs = a->q_hs;
    f.kc = a->kc;
    f.vc = a->vc;
    f.gate = a->gate;
    f.g_ts = a->g_ts;
    f.g_hs = a->g_hs;
    f.out = a->out;
    f.o_ts = a->o_ts;
    f.o_hs = a->o_hs;
    f.T = (int)a->T;
    f.off = (int)a->off;
    f.KV = (int)a->KV;
    f.ntq = (int)p.ntq;
    f.ct = (int)p.ct;
    f.max_splits = (int)p.max_splits;
    f.dyn = a->dyn;
    if (p.max_splits > 1) {
        f.part_acc = static_cast<float*>(a->ws);
        f.part_ml = reinterpret_cast<float*>(static_cast<char*>(a->ws) + p.acc_bytes);
    }
    const int64_t blocks = (int64_t)a->KV * p.ntq * p.max_splits;
    if (f.q16)
        bn_launch(ctx, (bn::flash_kernel<false>), dim3((unsigned)blocks), dim3(256), 0, st, f);
    else
        bn_launch(ctx, (bn::flash_kernel<true>), dim3((unsigned)blocks), dim3(256), 0, st, f);
    bn_status s = launched(ctx, "flash_kernel");
    if (s || p.max_splits == 1) return s;
    bn_launch(ctx, bn::flash_combine_kernel, dim3(a->T, a->H), dim3(64), 0, st, f);
    return launched(ctx, "flash_combine_kernel");
}

// The rotation of the gated output in place, after flash_kernel (the decode kernels and prefill_kernel rotate in
// their own epilogue).
bn_status rotate_in_place(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a) {
    bn::RotateArgs r{};
    r.attn = a->out;
    r.a_ts = a->o_ts;
    r.a_hs = a->o_hs;
    r.signs = a->signs;
    r.xr = a->out;
    r.x_ts = a->o_ts;
    r.x_hs = a->o_hs;
    r.T = (int)a->T;
    r.W = (int)a->H * bn::D;
    bn_launch(ctx, bn::rotate_kernel, dim3(a->T, a->H / 2), dim3(64), 0, st, r);
    return launched(ctx, "rotate_kernel");
}

// 17..64 rows that do not fill the GPU with prefill_kernel's q-tiles: verify_kernel over row groups of 8 rows (32
// query rows of a kv head per block, q read once per key split) after append_kernel writes the rows. flash_kernel
// has only one or two 32-token q-tiles per kv head there, so its parallelism comes from key splits that each reload
// the q-tile and write 128 rows of partials: measured 16.5 against 30 us for 33 rows over 5 cached keys (8/2 heads)
// and 36 against 71 us for 64 rows over 8,000 keys (16/4); from 100 rows up flash_kernel is faster (25 against
// 30 us at 100 rows over 300 keys, 28 against 33 us at 256 over 512), since each of its blocks stages a K/V tile
// once for 128 query rows where a row group uses it for 32. Keys per split: about kMidTargetBlocks blocks over the
// kv heads and row groups, whole 32-key tiles for each of the W waves.
constexpr int64_t kMidTargetBlocks = 256;
constexpr uint32_t kMidMaxRows = 64;
bool use_mid_rows(const bn_ctx* ctx, const bn_attn_args* a) {
    return ctx->mid_rows && a->T > (uint32_t)kVerifyMax && a->T <= kMidMaxRows &&
           !use_prefill(a, ctx->prefill_min_blocks);
}
int64_t mid_chunk(const bn_attn_args* a) {
    const int64_t T = a->T, nk = (int64_t)a->off + T, groups = ceil_div(T, 8);
    int64_t ns = ceil_div(kMidTargetBlocks, (int64_t)a->KV * groups);
    if (ns < 1) ns = 1;
    const int64_t step = 32 * BN_VERIFY_WAVES;
    return ceil_div(ceil_div(nk, ns), step) * step;
}
size_t mid_records_bytes(const bn_attn_args* a) {
    const int64_t T = a->T, ns = ceil_div((int64_t)a->off + T, mid_chunk(a));
    return (size_t)(a->KV * 8 * T * ceil_div(ns, 8)) * bn::DEC_PART * sizeof(float);
}

bn_status run_flash(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a) {
    if (use_mid_rows(ctx, a)) {
        bn_attn_args m = *a;
        if (a->k_new) {
            bn_status s = launch_append(ctx, st, a);
            if (s) return s;
            m.k_new = nullptr;
            m.v_new = nullptr;
        }
        return run_verify(ctx, st, &m, mid_chunk(a));
    }
    const bool fused = use_prefill(a, ctx->prefill_min_blocks);  // prefill_kernel rotates in its epilogue
    bn_status s = attend_flash(ctx, st, a);
    if (s || !a->signs || fused) return s;
    return rotate_in_place(ctx, st, a);
}

// prep_kernel over the rows of p; kv_only: K/V cache rows only (the attention kernel norms and rotates q itself)
bn_status launch_prep(bn_ctx* ctx, hipStream_t st, const bn_prep_args* a, bool kv_only) {
    bn::PrepArgs p{};
    p.qp = a->qp;
    p.qp_ts = a->qp_ts;
    p.qp_hs = a->qp_hs;
    p.kp = a->kp;
    p.vp = a->vp;
    p.rp.qn = a->q_norm;
    p.rp.kn = a->k_norm;
    p.rp.pos = a->pos;
    p.rp.inv_freq = a->inv_freq;
    p.rp.npos = (int)a->T;
    p.rp.rot = (int)a->rot;
    p.rp.s1 = (int)a->s1;
    p.rp.s2 = (int)a->s2;
    if (!kv_only) {
        if (a->flags & BN_Q_F16)
            p.q16 = static_cast<uint16_t*>(a->q);
        else
            p.q = static_cast<float*>(a->q);
    }
    p.q_ts = a->q_ts;
    p.q_hs = a->q_hs;
    p.kc = a->kc;
    p.vc = a->vc;
    p.dyn = a->dyn;
    p.T = (int)a->T;
    p.off = (int)a->off;
    p.H = (int)a->H;
    p.KV = (int)a->KV;
    // a few tokens (decode, verify): every 24 head rows of a token on a block of their own
    const int64_t rows = (kv_only ? 0 : a->H) + 2 * (int64_t)a->KV;
    if (a->T < 64)
        bn_launch(ctx, (bn::prep_kernel<8, 3>), dim3(a->T, (unsigned)ceil_div(rows, 24)), dim3(512), 0, st, p);
    else
        bn_launch(ctx, (bn::prep_kernel<4, 4>), dim3(a->T), dim3(256), 0, st, p);
    return launched(ctx, "prep_kernel");
}

// bn_attn_layer's arguments: p's checks (its q output needed only for more than kVerifyMax rows), a's q, k_new
// and v_new NULL, the same rows in both, and a's checks with p's raw rows in place of q, k_new and v_new (m).
bn_status check_layer(const bn_prep_args* p, const bn_attn_args* a, bn_attn_args* m, char* why) {
    if (!p || !a) return set_err(why, BN_EINVAL, "args is NULL");
    bn_status s = check_prep(p, why, p->T <= (uint32_t)kVerifyMax);
    if (s) return s;
    if (a->q || a->k_new || a->v_new)
        return set_err(why, BN_EINVAL, "q, k_new and v_new of the attention args must be NULL (the rows come from prep)");
    if (a->flags) return set_err(why, BN_EINVAL, "attention flags must be 0 (q's form is prep's flags)");
    if (p->T != a->T || p->off != a->off || p->H != a->H || p->KV != a->KV || p->cap != a->cap || p->kc != a->kc ||
        p->vc != a->vc || p->dyn != a->dyn)
        return set_err(why, BN_EINVAL, "prep and attention args describe different rows or caches");
    *m = *a;
    m->q = p->qp;
    m->q_ts = p->qp_ts;
    m->q_hs = p->qp_hs;
    m->k_new = p->kp;
    m->v_new = p->vp;
    return check_attn(m, 0, why);
}

bn_status check_kv_state(const bn_kv_state* s, char* why) {
    if (!s) return set_err(why, BN_EINVAL, "state is NULL");
    if (!s->kc || !s->vc || s->n_layers < 1 || s->KV < 1 || s->cap < 1)
        return set_err(why, BN_EINVAL, "kc, vc, n_layers, KV and cap are required");
    if (s->len > s->cap) return set_err(why, BN_EINVAL, "len %u exceeds cap %u", s->len, s->cap);
    if ((uint64_t)s->n_layers * s->cap * s->KV * bn::D > (uint64_t)1 << 46)
        return set_err(why, BN_EINVAL, "state too large");
    return BN_OK;
}

size_t kv_rows_bytes(const bn_kv_state* s, uint32_t len) { return (size_t)len * s->KV * bn::D * sizeof(uint16_t); }

void put_u32(uint8_t* p, uint32_t v) {
    for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i));
}
uint32_t get_u32(const uint8_t* p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

bn_status check_kv_section(const void* src, size_t bytes, const bn_kv_state* s, uint32_t* len_out, char* why) {
    bn_status st = check_kv_state(s, why);
    if (st) return st;
    if (!src || bytes < BN_KV_SECTION_HEADER) return set_err(why, BN_EINVAL, "section shorter than its header");
    const uint8_t* h = static_cast<const uint8_t*>(src);
    if (memcmp(h, BN_KV_SECTION_MAGIC, 8) != 0) return set_err(why, BN_EINVAL, "not a KV section (magic)");
    if (get_u32(h + 8) != BN_KV_SECTION_VERSION) return set_err(why, BN_EINVAL, "KV section version %u", get_u32(h + 8));
    if (get_u32(h + 12) != s->n_layers || get_u32(h + 16) != s->KV * (uint32_t)bn::D)
        return set_err(why, BN_EINVAL, "KV section of %u layers x %u values per row, state has %u x %u", get_u32(h + 12),
                       get_u32(h + 16), s->n_layers, s->KV * (uint32_t)bn::D);
    const uint32_t len = get_u32(h + 20);
    if (len > s->cap) return set_err(why, BN_EINVAL, "KV section of %u rows, cache holds %u", len, s->cap);
    const size_t need = BN_KV_SECTION_HEADER + 2 * (size_t)s->n_layers * kv_rows_bytes(s, len);
    if (bytes != need) return set_err(why, BN_EINVAL, "KV section of %zu bytes, %zu expected", bytes, need);
    if (len_out) *len_out = len;
    return BN_OK;
}

bn_status hip_err(bn_ctx* ctx, hipError_t e, const char* what) {
    if (e == hipSuccess) return BN_OK;
    return set_err(ctx->err, BN_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
}

bn_status check_ternary(const bn_ternary_args* a, char* why) {
    if (!a) return set_err(why, BN_EINVAL, "args is NULL");
    if (a->T < 1 || a->T > (1u << 24)) return set_err(why, BN_EINVAL, "T must be in 1..2^24 (T=%u)", a->T);
    if (a->k < 128 || (a->k & 127) || a->k > (1u << 20))
        return set_err(why, BN_EINVAL, "k must be a multiple of 128 in 128..2^20 (k=%u)", a->k);
    if (a->n_mats < 1 || a->n_mats > 3) return set_err(why, BN_EINVAL, "n_mats must be 1..3 (n_mats=%u)", a->n_mats);
    if (!a->x || !aligned16(a->x)) return set_err(why, BN_EINVAL, "x is required and must be 16-byte aligned");
    if (a->T > 1 && (a->x_ts < (int64_t)a->k || (a->x_ts & 3)))
        return set_err(why, BN_EINVAL, "x_ts must be a multiple of 4 and at least k");
    if (a->add > 1) return set_err(why, BN_EINVAL, "add must be 0 or 1");
    if (a->lora_r > 4096) return set_err(why, BN_EINVAL, "lora_r must be at most 4096");
    if (a->lora_r && (!a->lora_u || a->lora_us < 0 || (a->T > 1 && a->lora_us < (int64_t)a->n_mats * a->lora_r)))
        return set_err(why, BN_EINVAL, "lora_u is required with lora_r, lora_us at least n_mats * lora_r");
    int64_t rows = 0;
    for (uint32_t i = 0; i < a->n_mats; ++i) {
        const bn_ternary_mat& m = a->mat[i];
        if (!m.w || !m.s || !m.y) return set_err(why, BN_EINVAL, "mat[%u]: w, s and y are required", i);
        if (!aligned16(m.w) || ((uintptr_t)m.s & 1) || ((uintptr_t)m.y & 3) || ((uintptr_t)m.lora_b & 1))
            return set_err(why, BN_EINVAL, "mat[%u]: w must be 16-byte aligned, s, y and lora_b element aligned", i);
        if (m.o < 64 || (m.o & 63) || m.o > (1u << 24))
            return set_err(why, BN_EINVAL, "mat[%u]: o must be a multiple of 64 in 64..2^24 (o=%u)", i, m.o);
        if (a->T > 1 && m.y_ts < (int64_t)m.o) return set_err(why, BN_EINVAL, "mat[%u]: y_ts must be at least o", i);
        if (m.lora_b && !a->lora_r) return set_err(why, BN_EINVAL, "mat[%u]: lora_b given with lora_r = 0", i);
        rows += m.o;
    }
    if (rows > (1 << 30)) return set_err(why, BN_EINVAL, "too many rows");
    if (a->work && a->T > 32) {
        if ((uintptr_t)a->work & 255) return set_err(why, BN_EINVAL, "work must be 256-byte aligned");
        const uint64_t need = bn::tern_pf_work_bytes((int)a->T, (int)a->k);
        if (a->work_bytes < need)
            return set_err(why, BN_EINVAL, "work_bytes %llu below bn_ternary_workspace_size %llu",
                           (unsigned long long)a->work_bytes, (unsigned long long)need);
    }
    return BN_OK;
}

bn_status check_norm(const bn_norm_args* a, char* why) {
    if (!a) return set_err(why, BN_EINVAL, "args is NULL");
    if (a->T < 1 || a->T > (1u << 30)) return set_err(why, BN_EINVAL, "T must be in 1..2^30");
    if (a->d < 512 || (a->d & 511) || a->d > (1u << 16) * 512u)
        return set_err(why, BN_EINVAL, "d must be a multiple of 512 (d=%u)", a->d);
    if (!a->h || !a->w || !a->signs || !a->xr) return set_err(why, BN_EINVAL, "h, w, signs and xr are required");
    if (!aligned16(a->h) || !aligned16(a->w) || !aligned16(a->signs) || !aligned16(a->xr) || !aligned16(a->xn))
        return set_err(why, BN_EINVAL, "h, w, signs, xn and xr must be 16-byte aligned");
    if ((a->h_ts & 3) || (a->xr_ts & 3) || (a->xn && (a->xn_ts & 3)) ||
        (a->T > 1 && (a->h_ts < (int64_t)a->d || a->xr_ts < (int64_t)a->d || (a->xn && a->xn_ts < (int64_t)a->d))))
        return set_err(why, BN_EINVAL, "row strides must be multiples of 4, at least d");
    // the LoRA rows ride on the one-block-per-row kernel (d <= 8192)
    return check_lora(a->lora_a, a->lora_u, a->lora_us, a->lora_r, a->T, a->d, 16 * 512, why);
}

// tokens up to which the VALU rows kernel runs (4 or 8); more take the MFMA kernels
#ifndef BN_TERN_ROWS_MAX_T
#define BN_TERN_ROWS_MAX_T 4
#endif

// one-token calls with at least this many columns split each row group's words over two waves
#ifndef BN_TERN_ROWS_SPLIT_K
#define BN_TERN_ROWS_SPLIT_K 2048
#endif

// K split of the small-T MFMA kernel: 4 ways when each quarter of K is whole 64-column chunks, else 2 (k is a
// multiple of 128)
int tern_ksplit(uint32_t k) { return (k % (4 * bn::TERN_KC) == 0) ? 4 : 2; }

bn_status run_ternary(bn_ctx* ctx, hipStream_t st, const bn_ternary_args* a) {
    bn::TernArgs t{};
    int64_t rows = 0;
    for (uint32_t i = 0; i < 3; ++i) {
        const bn_ternary_mat& m = a->mat[i < a->n_mats ? i : 0];
        t.m[i].w = m.w;
        t.m[i].s = m.s;
        t.m[i].y = m.y;
        t.m[i].lb = m.lora_b;
        t.m[i].o = i < a->n_mats ? (int)m.o : 0;
        t.m[i].y_ts = m.y_ts;
        if (i < a->n_mats) rows += m.o;
    }
    t.n_mats = (int)a->n_mats;
    t.rows = (int)rows;
    t.x = a->x;
    t.x_ts = a->x_ts;
    t.T = (int)a->T;
    t.K = (int)a->k;
    t.add = (int)a->add;
    t.lu = a->lora_u;
    t.lu_ts = a->lora_us;
    t.lr = (int)a->lora_r;
    if (a->T <= BN_TERN_ROWS_MAX_T) {
        const dim3 grid((unsigned)ceil_div(rows, 4 * bn::TERN_ROWS_WAVE));
        switch (a->T) {
            case 1:
                // long rows: two waves split each row group's words (half the serial passes per wave)
                if (a->k >= BN_TERN_ROWS_SPLIT_K)
                    bn_launch(ctx, (bn::tern_rows_kernel<1, 2>), dim3((unsigned)ceil_div(rows, 2 * bn::TERN_ROWS_WAVE)),
                                       dim3(256), 0, st, t);
                else
                    bn_launch(ctx, bn::tern_rows_kernel<1>, grid, dim3(256), 0, st, t);
                break;
            case 2: bn_launch(ctx, bn::tern_rows_kernel<2>, grid, dim3(256), 0, st, t); break;
            case 3: bn_launch(ctx, bn::tern_rows_kernel<3>, grid, dim3(256), 0, st, t); break;
            case 4: bn_launch(ctx, bn::tern_rows_kernel<4>, grid, dim3(256), 0, st, t); break;
#if BN_TERN_ROWS_MAX_T > 4
            case 5: bn_launch(ctx, bn::tern_rows_kernel<5>, grid, dim3(256), 0, st, t); break;
            case 6: bn_launch(ctx, bn::tern_rows_kernel<6>, grid, dim3(256), 0, st, t); break;
            case 7: bn_launch(ctx, bn::tern_rows_kernel<7>, grid, dim3(256), 0, st, t); break;
            default: bn_launch(ctx, bn::tern_rows_kernel<8>, grid, dim3(256), 0, st, t); break;
#endif
        }
        return launched(ctx, "tern_rows_kernel");
    }
    if (a->T <= 32) {
        // one 32-token tile, 64 rows per block, K split over the block's waves
        const int row_tiles = (int)(rows / 64);
        const dim3 grid((unsigned)row_tiles);
        // fewer 64-row tiles than CUs (o_proj-sized matrices): 8 waves per block split K further
        if (row_tiles < ctx->cus && a->k % (8 * bn::TERN_KC) == 0)
            bn_launch(ctx, (bn::tern_mfma_kernel<1, 8, 1>), grid, dim3(512), 0, st, t, row_tiles);
        else if (tern_ksplit(a->k) == 4)
            bn_launch(ctx, (bn::tern_mfma_kernel<1, 4, 1>), grid, dim3(256), 0, st, t, row_tiles);
        else
            bn_launch(ctx, (bn::tern_mfma_kernel<1, 2, 1>), grid, dim3(128), 0, st, t, row_tiles);
        return launched(ctx, "tern_mfma_kernel<1>");
    }
    bool split_once = a->work != nullptr && bn::tern_pf_tiles((int)a->T, (int)a->k) <= (size_t)INT32_MAX;
    for (uint32_t i = 0; i < a->n_mats; ++i) split_once = split_once && !((uintptr_t)a->mat[i].s & 3);
    if (split_once) {
        // x split once into the workspace, then the GEMM streams it
        const size_t tiles = bn::tern_pf_tiles((int)a->T, (int)a->k);
        uint8_t* work = static_cast<uint8_t*>(a->work);
        bn_launch(ctx, bn::tern_split_kernel, dim3((unsigned)tiles), dim3(256), 0, st, a->x, a->x_ts, (int)a->T,
                           (int)a->k, work);
        const int row_tiles = (int)ceil_div(rows, 256);
        const int64_t blocks = (int64_t)row_tiles * ceil_div(a->T, bn::TPF_BM);
        if (blocks > INT32_MAX) return set_err(ctx->err, BN_EINVAL, "T * rows too large for one launch");
        // a grid of 64-token blocks that fits three per CU in one round runs as such (2 copy stages, three blocks
        // per CU); a larger one takes 128-token blocks (each decoded weight feeds twice the MFMAs; 2 stages, two
        // blocks per CU): the 4B q/k/v projection over 4,096 tokens 426-437 -> 387-405 us, same results bit for bit
        if (blocks <= 3 * (int64_t)ctx->cus)
            bn_launch(ctx, (bn::tern_pf_kernel<2, 3, 2>), dim3((unsigned)blocks), dim3(256), 0, st, t, row_tiles,
                               (const uint8_t*)work);
        else
            bn_launch(ctx, (bn::tern_pf_kernel<2, 2, 4>),
                      dim3((unsigned)(row_tiles * ceil_div(a->T, 2 * bn::TPF_BM))), dim3(256), 0, st, t, row_tiles,
                      (const uint8_t*)work);
        return launched(ctx, "tern_pf_kernel");
    }
    constexpr int MT = BN_TERN_PF_MT;
    constexpr int RG = BN_TERN_PF_RG;
    const int row_tiles = (int)ceil_div(rows, 64 * RG);
    const int64_t blocks = (int64_t)row_tiles * ceil_div(a->T, 32 * MT);
    if (blocks > INT32_MAX) return set_err(ctx->err, BN_EINVAL, "T * rows too large for one launch");
    bn_launch(ctx, (bn::tern_mfma_kernel<MT, 1, RG, BN_TERN_PF_OCC, BN_TERN_PF_KC>), dim3((unsigned)blocks),
                       dim3(64 * RG), 0, st, t, row_tiles);
    return launched(ctx, "tern_mfma_kernel (prefill)");
}

// The LoRA-A rows of an attention call, after it (a->lora_r > 0): lora_kernel rebuilds the gated rows from `out`.
bn_status launch_lora(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a) {
    if (!a->lora_r) return BN_OK;
    bn::LoraOutArgs l{};
    l.l.A = a->lora_a;
    l.l.U = a->lora_u;
    l.l.u_ts = a->lora_us;
    l.l.R = (int)a->lora_r;
    l.l.rpb = a->T >= 64 ? 32 : 8;
    l.out = a->out;
    l.o_ts = a->o_ts;
    l.o_hs = a->o_hs;
    l.signs = a->signs;
    l.W = (int)a->H * bn::D;
    bn_launch(ctx, bn::lora_kernel, dim3(a->T, (unsigned)ceil_div(a->lora_r, l.l.rpb)), dim3(256),
                       (size_t)l.W * sizeof(float), st, l);
    return launched(ctx, "lora_kernel");
}

// kind: 0 forward, 1 decode, 2 verify, 3 prefill. One row is always a decode; verify-sized calls (T <= 16) of the
// forward and verify entry points run as decodes of their rows; the rest take the MFMA prefill kernels. Then the
// LoRA-A rows, when asked for.
bn_status run(bn_ctx* ctx, hipStream_t st, const bn_attn_args* a, int kind) {
    bn_status s;
    const int64_t chunk = (kind != 3 && ctx->verify_mfma) ? verify_chunk(a) : 0;
    if (chunk)
        s = run_verify(ctx, st, a, chunk);
    else if (a->T == 1 || (kind != 3 && a->T <= (uint32_t)kVerifyMax))
        s = run_rows(ctx, st, a);
    else
        s = run_flash(ctx, st, a);
    return s ? s : launch_lora(ctx, st, a);
}

// The ragged decode with its partials in `ws` (the caller's workspace, or this device's `scratch`).
bn_status run_ragged(bn_ctx* ctx, hipStream_t st, const bn_ragged_args* a, const DecodePlan& p, void* ws) {
    bn::DecodeArgs d{};
    d.q = a->q;
    d.q_ss = a->q_ss;
    d.q_hs = a->q_hs;
    d.k_new = a->k_new;
    d.v_new = a->v_new;
    d.kn_ss = (int64_t)a->KV * bn::D;
    d.kc = a->kc;
    d.vc = a->vc;
    d.kv_off = a->kv_off;
    d.kv_len = a->kv_len;
    d.gate = a->gate;
    d.g_ss = a->g_ss;
    d.g_hs = a->g_hs;
    d.out = a->out;
    d.o_ss = a->o_ss;
    d.o_hs = a->o_hs;
    d.signs = a->signs;
    d.KV = (int)a->KV;
    bind_workspace(d, p, ws);
    return launch_decode(ctx, st, d, p);
}

}  // namespace

extern "C" {

int bn_abi_version(void) { return BN_ABI_VERSION; }

bn_status bn_dyn_overflow(bn_ctx* ctx, int* flag) {
    if (!ctx || !flag) return BN_EINVAL;
    int prev = -1;
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (hipSetDevice(ctx->device) != hipSuccess) return set_err(ctx->err, BN_EDEVICE, "hipSetDevice failed");
    unsigned int v = 0;
    const unsigned int zero = 0;
    hipError_t e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(bn::dyn_overflow), sizeof(v), 0, hipMemcpyDeviceToHost);
    if (e == hipSuccess && v) e = hipMemcpyToSymbol(HIP_SYMBOL(bn::dyn_overflow), &zero, sizeof(zero), 0,
                                                    hipMemcpyHostToDevice);
    if (prev >= 0 && prev != ctx->device) (void)hipSetDevice(prev);
    if (e != hipSuccess) return set_err(ctx->err, BN_EDEVICE, "dyn overflow flag: %s", hipGetErrorString(e));
    *flag = v != 0;
    return BN_OK;
}

const char* bn_status_str(bn_status s) {
    switch (s) {
        case BN_OK: return "ok";
        case BN_EINVAL: return "invalid argument";
        case BN_ENOWS: return "workspace too small";
        case BN_ELAUNCH: return "kernel launch failed";
        case BN_EDEVICE: return "device error";
    }
    return "unknown status";
}

bn_status bn_ctx_create(int device, bn_ctx** out) {
    if (!out) return BN_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return BN_EDEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return BN_EDEVICE;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return BN_EDEVICE;
    bn_ctx* c = new (std::nothrow) bn_ctx;
    if (!c) return BN_EDEVICE;
    c->device = device;
    c->cus = prop.multiProcessorCount;
    c->prefill_min_blocks = c->cus;
    if (const char* e = getenv("BONSAI_ATTN_PREFILL_MIN_BLOCKS")) {
        const int v = atoi(e);
        if (v >= 1) c->prefill_min_blocks = v;
    }
    c->decode_waves = BN_DECODE_WAVES;
    if (const char* e = getenv("BONSAI_ATTN_DECODE_WAVES")) {
        const int v = atoi(e);
        if (v == 1 || v == 2 || v == 4 || v == 8) c->decode_waves = v;
    }
    c->decode_target_waves = BN_DECODE_TARGET_WAVES;
    if (const char* e = getenv("BONSAI_ATTN_DECODE_TARGET_WAVES")) {
        const int v = atoi(e);
        if (v >= 256 && v <= BN_DECODE_MAX_TARGET_WAVES) c->decode_target_waves = v;
    }
    c->decode_max_splits = BN_DECODE_MAX_SPLITS;
    if (const char* e = getenv("BONSAI_ATTN_DECODE_MAX_SPLITS")) {
        const int v = atoi(e);
        if (v >= 1 && v <= kMaxSplitsCap) c->decode_max_splits = v;
    }
    c->flash_target_blocks = (int)kFlashTargetBlocks;
    if (const char* e = getenv("BONSAI_ATTN_FLASH_TARGET_BLOCKS")) {
        const int v = atoi(e);
        if (v >= 1 && v <= kFlashTargetBlocks) c->flash_target_blocks = v;
    }
    c->verify_mfma = 1;
    if (const char* e = getenv("BONSAI_ATTN_VERIFY_MFMA")) c->verify_mfma = atoi(e) != 0;
    c->prefill_pair = 0;
    if (const char* e = getenv("BONSAI_ATTN_PREFILL_PAIR")) c->prefill_pair = atoi(e) != 0;
    c->mid_rows = 1;
    if (const char* e = getenv("BONSAI_ATTN_MID_ROWS")) c->mid_rows = atoi(e) != 0;
    c->scratch = scratch_address(device);
    c->launch_err = hipSuccess;
    c->err[0] = 0;
    *out = c;
    return BN_OK;
}

void bn_ctx_destroy(bn_ctx* ctx) { delete ctx; }

const char* bn_ctx_last_error(const bn_ctx* ctx) { return ctx ? ctx->err : g_check_err; }

size_t bn_attn_workspace_size(const bn_attn_args* a) {
    if (!a || a->KV < 1 || a->T < 1) return 0;
    size_t rows = a->T <= (uint32_t)kVerifyMax ? plan_rows(a, 1, BN_DECODE_MAX_TARGET_WAVES, kMaxSplitsCap).total() : 0;
    if (verify_chunk(a)) rows = verify_q_offset(a) + (size_t)a->T * a->H * bn::D * sizeof(float);
    if (a->T == 1) return rows;
    // the kernel choice for T >= 2 depends on the context, so the size covers the flash kernel's partials and, for
    // more than 16 rows, verify_kernel's row-group records
    size_t fl = plan_flash(a->T, a->off, a->KV).total();
    if (a->T > (uint32_t)kVerifyMax && a->T <= kMidMaxRows) {
        const size_t mid = mid_records_bytes(a);
        if (mid > fl) fl = mid;
    }
    return fl > rows ? fl : rows;
}

size_t bn_ragged_workspace_size(const bn_ragged_args* a) {
    if (!a || a->KV < 1 || a->nseq < 1 || a->max_len < 1) return 0;
    return plan_decode(a->nseq, a->KV, a->max_len, -1, 1, BN_DECODE_MAX_TARGET_WAVES, kMaxSplitsCap).total();
}

bn_status bn_attn_check(const bn_attn_args* a, int kind) { return check_attn(a, kind, g_check_err); }

bn_status bn_ragged_check(const bn_ragged_args* a) { return check_ragged(a, g_check_err); }

bn_status bn_workspace_clear(bn_ctx* ctx, bn_stream stream, void* ws, size_t bytes) {
    if (!ctx) return BN_EINVAL;
    if (!bytes) return BN_OK;
    if (!ws || !aligned16(ws)) return set_err(ctx->err, BN_EINVAL, "workspace must be 16-byte aligned");
    int64_t n16 = (int64_t)(bytes / 16);
    int ntail = (int)(bytes % 16);
    int64_t blocks = ceil_div(n16 > 0 ? n16 : 1, 256);
    if (blocks > 2048) blocks = 2048;
    bn_launch(ctx, bn::fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       static_cast<bn::u4*>(ws), n16, static_cast<uint8_t*>(ws) + n16 * 16, ntail);
    return launched(ctx, "fill_zero_kernel");
}

bn_status bn_attn_append(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_attn(a, 4, ctx->err);
    if (s) return s;
    return launch_append(ctx, (hipStream_t)stream, a);
}

bn_status bn_attn_decode(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_attn(a, 1, ctx->err);
    if (s) return s;
    return run(ctx, (hipStream_t)stream, a, 1);
}

bn_status bn_attn_verify(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_attn(a, 2, ctx->err);
    if (s) return s;
    return run(ctx, (hipStream_t)stream, a, 2);
}

bn_status bn_attn_prefill(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_attn(a, 3, ctx->err);
    if (s) return s;
    return run(ctx, (hipStream_t)stream, a, 3);
}

bn_status bn_attn_forward(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_attn(a, 0, ctx->err);
    if (s) return s;
    return run(ctx, (hipStream_t)stream, a, 0);
}

bn_status bn_attn_decode_ragged(bn_ctx* ctx, bn_stream stream, const bn_ragged_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_ragged(a, ctx->err);
    if (s) return s;
    const DecodePlan p = plan_decode(a->nseq, a->KV, a->max_len, -1, ctx->decode_waves, ctx->decode_target_waves,
                                     ctx->decode_max_splits);
    return run_ragged(ctx, (hipStream_t)stream, a, p, a->ws);
}

bn_status bn_attn_decode_ragged_noalloc(bn_ctx* ctx, bn_stream stream, const bn_ragged_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_ragged(a, ctx->err, false);
    if (s) return s;
    if (!ctx->scratch) return set_err(ctx->err, BN_EDEVICE, "the device address of the scratch array is unavailable");
    const DecodePlan p = plan_decode(a->nseq, a->KV, a->max_len, -1, ctx->decode_waves, ctx->decode_target_waves,
                                     ctx->decode_max_splits);
    if (p.total() > BN_NOALLOC_SCRATCH_BYTES)
        return set_err(ctx->err, BN_ENOWS, "the partials of this batch need %zu bytes, the scratch array holds %u",
                       p.total(), BN_NOALLOC_SCRATCH_BYTES);
    return run_ragged(ctx, (hipStream_t)stream, a, p, ctx->scratch);
}

bn_status bn_kv_copy(bn_ctx* ctx, bn_stream stream, const bn_kv_state* from, const bn_kv_state* to) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_kv_state(from, ctx->err);
    if (!s) s = check_kv_state(to, ctx->err);
    if (s) return s;
    if (from->n_layers != to->n_layers || from->KV != to->KV)
        return set_err(ctx->err, BN_EINVAL, "states of different shapes");
    if (from->len > to->cap) return set_err(ctx->err, BN_EINVAL, "len %u exceeds the target's cap %u", from->len, to->cap);
    if (from->len == 0) return BN_OK;
    if (!aligned16(from->kc) || !aligned16(from->vc) || !aligned16(to->kc) || !aligned16(to->vc)) {
        // caches not 16-byte aligned: the runtime's 2-D copies
        const size_t w = kv_rows_bytes(from, from->len);
        const size_t sp = kv_rows_bytes(from, from->cap), dp = kv_rows_bytes(to, to->cap);
        hipError_t e = hipMemcpy2DAsync(to->kc, dp, from->kc, sp, w, from->n_layers, hipMemcpyDeviceToDevice,
                                        (hipStream_t)stream);
        if (e == hipSuccess)
            e = hipMemcpy2DAsync(to->vc, dp, from->vc, sp, w, from->n_layers, hipMemcpyDeviceToDevice,
                                 (hipStream_t)stream);
        return hip_err(ctx, e, "KV copy");
    }
    // rows are KV * 512 bytes, so a layer's used rows and the layer pitches are whole 16-byte groups
    const int64_t w16 = (int64_t)(kv_rows_bytes(from, from->len) / 16);
    const int64_t sp16 = (int64_t)(kv_rows_bytes(from, from->cap) / 16), dp16 = (int64_t)(kv_rows_bytes(to, to->cap) / 16);
    const int64_t cpl = ceil_div(w16, 256 * bn::KVC_U), chunks = 2 * (int64_t)from->n_layers * cpl;
    // the dispatch counts work-items in 32 bits: at most 2^24 - 1 blocks of 256 (a 256 GiB copy)
    if (chunks > (int64_t)(UINT32_MAX / 256)) return set_err(ctx->err, BN_EINVAL, "KV copy too large for one launch");
    bn_launch(ctx, bn::kv_copy_kernel, dim3((unsigned)chunks), dim3(256), 0,
              (hipStream_t)stream, reinterpret_cast<const bn::u4*>(from->kc), reinterpret_cast<const bn::u4*>(from->vc),
              reinterpret_cast<bn::u4*>(to->kc), reinterpret_cast<bn::u4*>(to->vc), w16, sp16, dp16,
              (int)from->n_layers, (int)cpl);
    return launched(ctx, "kv_copy_kernel");
}

size_t bn_kv_section_size(const bn_kv_state* s) {
    char why[256];
    if (check_kv_state(s, why)) return 0;
    return BN_KV_SECTION_HEADER + 2 * (size_t)s->n_layers * kv_rows_bytes(s, s->len);
}

bn_status bn_kv_section_save(bn_ctx* ctx, bn_stream stream, const bn_kv_state* s, void* dst, size_t dst_bytes) {
    if (!ctx) return BN_EINVAL;
    bn_status st = check_kv_state(s, ctx->err);
    if (st) return st;
    const size_t need = bn_kv_section_size(s);
    if (!dst || dst_bytes < need) return set_err(ctx->err, BN_EINVAL, "section needs %zu bytes", need);
    uint8_t* h = static_cast<uint8_t*>(dst);
    memcpy(h, BN_KV_SECTION_MAGIC, 8);
    put_u32(h + 8, BN_KV_SECTION_VERSION);
    put_u32(h + 12, s->n_layers);
    put_u32(h + 16, s->KV * (uint32_t)bn::D);
    put_u32(h + 20, s->len);
    const size_t rb = kv_rows_bytes(s, s->len), lp = kv_rows_bytes(s, s->cap);
    hipError_t e = hipSuccess;
    if (rb) {
        uint8_t* body = h + BN_KV_SECTION_HEADER;
        e = hipMemcpy2DAsync(body, rb, s->kc, lp, rb, s->n_layers, hipMemcpyDeviceToHost, (hipStream_t)stream);
        if (e == hipSuccess)
            e = hipMemcpy2DAsync(body + s->n_layers * rb, rb, s->vc, lp, rb, s->n_layers, hipMemcpyDeviceToHost,
                                 (hipStream_t)stream);
        if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    }
    return hip_err(ctx, e, "KV section save");
}

bn_status bn_kv_section_check(const void* src, size_t src_bytes, const bn_kv_state* s, uint32_t* len_out) {
    return check_kv_section(src, src_bytes, s, len_out, g_check_err);
}

bn_status bn_kv_section_load(bn_ctx* ctx, bn_stream stream, const void* src, size_t src_bytes, const bn_kv_state* s,
                             uint32_t* len_out) {
    if (!ctx) return BN_EINVAL;
    uint32_t len = 0;
    bn_status st = check_kv_section(src, src_bytes, s, &len, ctx->err);
    if (st) return st;
    const size_t rb = kv_rows_bytes(s, len), lp = kv_rows_bytes(s, s->cap);
    hipError_t e = hipSuccess;
    if (rb) {
        const uint8_t* body = static_cast<const uint8_t*>(src) + BN_KV_SECTION_HEADER;
        e = hipMemcpy2DAsync(s->kc, lp, body, rb, rb, s->n_layers, hipMemcpyHostToDevice, (hipStream_t)stream);
        if (e == hipSuccess)
            e = hipMemcpy2DAsync(s->vc, lp, body + s->n_layers * rb, rb, rb, s->n_layers, hipMemcpyHostToDevice,
                                 (hipStream_t)stream);
        if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    }
    st = hip_err(ctx, e, "KV section load");
    if (!st && len_out) *len_out = len;
    return st;
}

bn_status bn_prep_check(const bn_prep_args* a) { return check_prep(a, g_check_err); }

bn_status bn_layer_check(const bn_prep_args* p, const bn_attn_args* a) {
    bn_attn_args m;
    return check_layer(p, a, &m, g_check_err);
}

bn_status bn_rotate_check(const bn_rotate_args* a) { return check_rotate(a, g_check_err); }

bn_status bn_attn_prep(bn_ctx* ctx, bn_stream stream, const bn_prep_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_prep(a, ctx->err);
    if (s) return s;
    return launch_prep(ctx, (hipStream_t)stream, a, false);
}

bn_status bn_attn_layer(bn_ctx* ctx, bn_stream stream, const bn_prep_args* p, const bn_attn_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_attn_args m;
    bn_status s = check_layer(p, a, &m, ctx->err);
    if (s) return s;
    hipStream_t st = (hipStream_t)stream;
    bn::RopeParams rp{};
    rp.qn = p->q_norm;
    rp.kn = p->k_norm;
    rp.pos = p->pos;
    rp.inv_freq = p->inv_freq;
    rp.npos = (int)p->T;
    rp.rot = (int)p->rot;
    rp.s1 = (int)p->s1;
    rp.s2 = (int)p->s2;
    if (p->T <= (uint32_t)kVerifyMax) {
        // 2..16 rows: prep_kernel writes q (to p->q in its form, else fp32 into the workspace after the partials)
        // and the K/V rows, then verify_kernel and the merge
        const int64_t chunk = ctx->verify_mfma ? verify_chunk(&m) : 0;
        if (chunk) {
            bn_prep_args pq = *p;
            if (!pq.q) {
                pq.q = static_cast<char*>(m.ws) + verify_q_offset(&m);
                pq.flags = 0;
                pq.q_ts = (int64_t)p->H * bn::D;
                pq.q_hs = bn::D;
            }
            s = launch_prep(ctx, st, &pq, false);
            if (s) return s;
            m.k_new = nullptr;
            m.v_new = nullptr;
            m.q = pq.q;
            m.q_ts = pq.q_ts;
            m.q_hs = pq.q_hs;
            m.flags = pq.flags;
            s = run_verify(ctx, st, &m, chunk);
            return s ? s : launch_lora(ctx, st, &m);
        }
        // decode / verify rows: q normed and rotated in the split kernel's prologue; one row also appends its
        // K/V row there, several rows have theirs written by prep_kernel first
        if (p->T > 1) {
            s = launch_prep(ctx, st, p, true);
            if (s) return s;
            m.k_new = nullptr;
            m.v_new = nullptr;
        }
        s = run_rows(ctx, st, &m, &rp);
        return s ? s : launch_lora(ctx, st, &m);
    }
    // prefill: prep_kernel writes q (to p->q, fp16 with BN_Q_F16) and the K/V rows, then the prefill kernels read
    // them (norming q inside prefill_kernel's Q staging was measured slower: 252 against 240 us at 4096 rows,
    // the staging sits on every block's critical path)
    s = launch_prep(ctx, st, p, false);
    if (s) return s;
    m.k_new = nullptr;
    m.v_new = nullptr;
    m.q = p->q;
    m.q_ts = p->q_ts;
    m.q_hs = p->q_hs;
    m.flags = p->flags;
    s = run_flash(ctx, st, &m);
    return s ? s : launch_lora(ctx, st, &m);
}

bn_status bn_ternary_check(const bn_ternary_args* a) { return check_ternary(a, g_check_err); }
size_t bn_ternary_workspace_size(uint32_t T, uint32_t k) {
    return (T > 32 && k >= 128 && !(k & 127)) ? bn::tern_pf_work_bytes((int)T, (int)k) : 0;
}

bn_status bn_norm_check(const bn_norm_args* a) { return check_norm(a, g_check_err); }

bn_status bn_norm_rotate(bn_ctx* ctx, bn_stream stream, const bn_norm_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_norm(a, ctx->err);
    if (s) return s;
    bn::NormRotateArgs n{};
    n.h = a->h;
    n.h_ts = a->h_ts;
    n.w = a->w;
    n.signs = a->signs;
    n.xn = a->xn;
    n.xn_ts = a->xn_ts;
    n.xr = a->xr;
    n.xr_ts = a->xr_ts;
    n.T = (int)a->T;
    n.D = (int)a->d;
    if (a->d <= 16 * 512) {
        // LoRA rows: extra blocks of the launch, each with the row staged in LDS and rpb rows of u over its waves
        const int waves = (int)(a->d / 512);
        n.lora.A = a->lora_a;
        n.lora.U = a->lora_u;
        n.lora.u_ts = a->lora_us;
        n.lora.R = (int)a->lora_r;
        n.lora.rpb = waves * (a->T >= 64 ? 4 : 1);
        const unsigned extra = a->lora_r ? (unsigned)ceil_div(a->lora_r, n.lora.rpb) : 0u;
        bn_launch(ctx, bn::norm_rotate_row_kernel, dim3(a->T, 1 + extra), dim3(64 * waves),
                           a->lora_r ? (size_t)a->d * sizeof(float) : 0, (hipStream_t)stream, n);
        return launched(ctx, "norm_rotate_row_kernel");
    }
    bn_launch(ctx, bn::norm_rotate_kernel, dim3(a->T, a->d / 512), dim3(64), 0, (hipStream_t)stream, n);
    return launched(ctx, "norm_rotate_kernel");
}

bn_status bn_ternary_matmul(bn_ctx* ctx, bn_stream stream, const bn_ternary_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_ternary(a, ctx->err);
    if (s) return s;
    return run_ternary(ctx, (hipStream_t)stream, a);
}

bn_status bn_gate_rotate(bn_ctx* ctx, bn_stream stream, const bn_rotate_args* a) {
    if (!ctx) return BN_EINVAL;
    bn_status s = check_rotate(a, ctx->err);
    if (s) return s;
    bn::RotateArgs r{};
    r.attn = a->attn;
    r.a_ts = a->a_ts;
    r.a_hs = bn::D;
    r.gate = a->gate;
    r.g_ts = a->g_ts;
    r.g_hs = a->g_hs;
    r.signs = a->signs;
    r.xr = a->xr;
    r.x_ts = a->x_ts;
    r.x_hs = bn::D;
    r.T = (int)a->T;
    r.W = (int)a->H * bn::D;
    // LoRA rows: extra blocks of the launch, each staging the gated row in LDS for rpb rows of u
    r.lora.A = a->lora_a;
    r.lora.U = a->lora_u;
    r.lora.u_ts = a->lora_us;
    r.lora.R = (int)a->lora_r;
    r.lora.rpb = a->T >= 64 ? 16 : 4;
    const unsigned extra = a->lora_r ? (unsigned)ceil_div(a->lora_r, r.lora.rpb) : 0u;
    bn_launch(ctx, bn::rotate_kernel, dim3(a->T, a->H / 2 + extra), dim3(64),
                       a->lora_r ? (size_t)r.W * sizeof(float) : 0, (hipStream_t)stream, r);
    return launched(ctx, "rotate_kernel");
}

}  // extern "C"
