// Causal GQA prefill for long prompts on fp16 MFMA: 8 waves per block, the key range of every q-tile split
// between two wave groups that merge through LDS.
//
// Semantics follow attn_split.comp:9-58 + attn_combine.comp:6-21 + gate_rotate.comp:19-25 of the reference:
// row t (position off+t) of head h attends to cache rows [0, off+t+1) of kv head h/4; softmax(q.k/16) v,
// then a * sigmoid(gate). The K/V rows of the call are appended to the cache before this kernel runs.
//
// Decomposition (this kernel's own):
//   A q-tile is 32 consecutive tokens of the 4 query heads of one kv head (128 query rows); one block per
//   q-tile. The block's 8 waves form two groups of 4 (one wave per query head, 32 rows each). Group 0 attends
//   to the first half of the q-tile's key tiles, group 1 to the second half, each with its own double-buffered
//   K/V stages in LDS; at the end the two partial (m, l, O) are merged through LDS in group order. Waves w and
//   w+4 share a SIMD, so one wave's softmax (VALU) overlaps the other's MFMAs.
//   Splitting the key range inside the block is what balances the causal triangle: a 4096-token prompt has
//   exactly as many query rows as 256 CUs x 8 waves x 32 rows hold, so whole q-tiles per CU would leave the
//   short ones idle half the time; with the split a block's cost is half its key range, and blocks issued
//   longest first pair up (long + short) on each CU.
//   K/V tiles of 32 keys are copied HBM/L2 -> LDS by global_load_lds (no VGPRs). Rows p and p+16 of a tile
//   share one 1 KB copy instruction; the pairs are padded (K: 16 B, V: 64 B per pair) so the K operand reads
//   (16 rows x 16 B per 16 lanes) and the transposed V reads (4 rows x 64 B per 32 lanes) fall on distinct
//   banks, and every LDS address is one per-lane base register plus an immediate. A wave's 8 copies of the next
//   tile are issued one after each pair of the current tile's S^T MFMAs, not as a burst before them.
//   S^T = K Q^T on v_mfma_f32_32x32x16_f16 (A = K from LDS, B = Q^T in registers; q comes as fp16 bits, an fp32
//   q goes to prefill_hilo_kernel, which keeps its precision). Softmax in fp32, log2
//   domain; the running max moves only when a row's max grows by more than 2^8, so O is rarely rescaled. The
//   row sums add the fp16-rounded probabilities (v_dot2_f32_f16), the same values the PV product uses.
//   O += P V with P straight from the S^T registers (A operand) and V from two ds_read_b64_tr_b16 reads that
//   fetch exactly the keys those registers hold.
//   Causal masking only on tiles that cross the diagonal; tiles past it are not visited.
//   Block order: longest q-tiles first, each kv head pinned to a fixed set of XCDs.
#pragma once
#include <type_traits>

#include "bn_device.h"

namespace bn {

constexpr int PF_BQ = 32;                 // tokens per q-tile (rows per wave)
constexpr int PF_BK = 32;                 // keys per K/V tile
constexpr int PF_KP = 1040;               // bytes per K row pair (rows p, p+16) in LDS
constexpr int PF_VP = 1088;               // bytes per V row pair
constexpr int PF_KB = 16 * PF_KP;         // K tile bytes
constexpr int PF_VB = 16 * PF_VP;         // V tile bytes
constexpr int PF_STAGE = PF_KB + PF_VB;   // one K + V stage (34,048 B)
constexpr int PF_XSLOT = 16384;           // O exchange per wave at the end: 4 tiles of 32 x 32 fp32
constexpr int PF_QP = 528;                // row pitch of prefill_pair_kernel's fp16 Q staging rows in LDS

struct PrefillArgs {
    const float* q;          // element t*q_ts + h*q_hs + d (fp32: prefill_hilo_kernel) ...
    const uint16_t* q16;     // ... or fp16 bits (prefill_kernel)
    int64_t q_ts, q_hs;
    const uint16_t* kc;      // fp16 [rows][KV][256]
    const uint16_t* vc;
    const float* gate;       // element t*g_ts + h*g_hs + d, or null
    int64_t g_ts, g_hs;
    float* out;              // element t*o_ts + h*o_hs + d
    int64_t o_ts, o_hs;
    const float* signs;      // [heads*256] +-1, or null: out receives each row rotated (blocks of 512 = heads
                             // 2j, 2j+1, times the signs, Walsh-Hadamard transformed, / sqrt(512))
    const uint32_t* dyn;     // device offset (graph replay) or null; off is then its upper bound
    int T, off, KV, ntq;
};

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef short pf_s4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pf_s4v pf_lds_s4_t;
typedef __attribute__((address_space(3))) void pf_lds_void_t;

__device__ __forceinline__ h8 pf_lds_h8(const uint8_t* p) { return *reinterpret_cast<const h8*>(p); }
__device__ __forceinline__ h4 pf_lds_tr(const uint8_t* p) {
    return __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_s4_t*)(p)));
}
__device__ __forceinline__ void pf_wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// 16 bytes per lane from global memory into LDS at lds_base + 16 lane (global_load_lds_dwordx4), written as
// assembly so that the compiler does not track it: its own tracking of these copies cannot tell the stages (or the
// K and V halves) of one LDS array apart and would wait for every copy in flight before each operand read. The
// caller orders the copies against the reads itself (s_waitcnt vmcnt, then a wave or block barrier). M0 carries the
// LDS base; nothing else in the kernels that use this sets M0.
__device__ __forceinline__ void pf_copy16(const void* g, const uint8_t* lds_base) {
    const uint32_t la = (uint32_t)(uintptr_t)(pf_lds_void_t*)lds_base;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(la) : "memory");
}

__global__ __launch_bounds__(512) void prefill_kernel(PrefillArgs a) {
    // stage 0 and stage 1 of both groups are separate LDS objects: the compiler then sees that a tile copy into
    // one stage cannot alias reads of the other, and does not wait for the copy before those reads
    __shared__ __attribute__((aligned(1024))) uint8_t lds_s0[2 * PF_STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_s1[2 * PF_STAGE];
    __shared__ float ml_lds[2][4][2][32];  // per group, wave: m, l of the wave's 32 rows
    __shared__ f4 bc_lds[8][16];           // per wave: up to 64 floats broadcast in row order

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), g = wave >> 2, w = wave & 3;  // wave-uniform
    const int h = lane >> 5, r32 = lane & 31;
    const int KV = a.KV, ntq = a.ntq;
    // every argument word the block needs is requested at entry, in one round trip (left alone, the compiler
    // fetches them in several dependent batches before the first copy goes out)
    asm volatile("" ::"s"(a.q16), "s"(a.q_ts), "s"(a.q_hs), "s"(a.kc), "s"(a.vc), "s"(a.gate), "s"(a.g_ts),
                 "s"(a.g_hs), "s"(a.out), "s"(a.o_ts), "s"(a.o_hs), "s"(a.signs), "s"(a.dyn), "s"(a.T), "s"(a.off));

    // block -> (kv head, q-tile): longest q-tiles (highest index) first
    int kh, qt;
    {
        const int b = blockIdx.x, nb = KV * ntq;
        int idx;
        if (8 % KV == 0 && nb % 8 == 0) {
            // XCD x (= b % 8) serves kv head x % KV
            const int xcd = b & 7, reps = 8 / KV;
            kh = xcd % KV;
            idx = (b >> 3) * reps + xcd / KV;
        } else {
            kh = b % KV;
            idx = b / KV;
        }
        qt = ntq - 1 - idx;
    }
    const int t0 = qt * PF_BQ;
    const int t_last = min(a.T, t0 + PF_BQ) - 1;
    const int off = call_off(a.dyn, a.off);
    const int nk = off + a.T;                            // cache rows that exist
    const int nt = (off + t_last + PF_BK) / PF_BK;       // key tiles the q-tile attends to
    const int half = (nt + 1) >> 1;
    const int j_begin = g ? half : 0, j_end = g ? nt : half;
    const int64_t kvd = (int64_t)KV * D;
    const uint16_t* kb = a.kc + (int64_t)kh * D;
    const uint16_t* vb = a.vc + (int64_t)kh * D;
    const int head = kh * 4 + w;

    // Q rows of the block (4 heads x 32 tokens, fp16) are copied by global_load_lds into the free second stage of
    // each group (heads 0-1 in group 0's, heads 2-3 in group 1's) in a K tile's layout: rows p and p+16 of a head in
    // one 1 KB copy, pairs PF_KP apart, so the Q^T operand reads are the K operand reads' conflict-free pattern. Wave w
    // copies pairs 8 (w % 2) .. +7 of head w / 2. No VGPRs and no wait before the first K/V tile's copies go out too.
    auto q_stage = [&](int hq) -> uint8_t* { return lds_s1 + (hq >> 1) * PF_STAGE + (hq & 1) * 16 * PF_KP; };
    {
        const int hq = wave >> 1;
        const uint16_t* qh = a.q16 + (int64_t)(kh * 4 + hq) * a.q_hs + 8 * r32;
        uint8_t* const qs = q_stage(hq);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int p = 8 * (wave & 1) + i;
            const int tl = min(t0 + p + 16 * h, a.T - 1);
            __builtin_amdgcn_global_load_lds(qh + (int64_t)tl * a.q_ts, (pf_lds_void_t*)(qs + p * PF_KP), 16, 0, 0);
        }
    }

    // Tile copy (per group): wave w moves row pairs 4w .. 4w+3 of K and of V; lane l of an instruction loads
    // row p + 16*(l/32), 16-byte chunk l%32, into LDS pair p at byte 16*l. The tile base is wave-uniform; rows past
    // the cache's last row are clamped to it per lane (their scores are masked). No branch: the copies of the next
    // tile sit in the same basic block as the current tile's S product, where they are interleaved with its MFMAs.
    const uint32_t lane_go = (uint32_t)(r32 * 8) * 2u;
    auto issue_tile = [&](int j, uint8_t* st) {
        const int j0 = j * PF_BK, lim = nk - 1 - j0;  // last valid row of this tile
        const char* kt = reinterpret_cast<const char*>(kb + (int64_t)j0 * kvd);
        const char* vt = reinterpret_cast<const char*>(vb + (int64_t)j0 * kvd);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = 4 * w + i;
            const uint32_t go = (uint32_t)(min(p + 16 * h, lim) * (int)kvd) * 2u + lane_go;
            __builtin_amdgcn_global_load_lds(kt + go, (pf_lds_void_t*)(st + p * PF_KP), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vt + go, (pf_lds_void_t*)(st + PF_KB + p * PF_VP), 16, 0, 0);
        }
    };

    f16x o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float sc = QK_SCALE * LOG2E;
    const int qpos = off + t0 + r32;  // this lane's row sees keys <= qpos

    // per-lane LDS bases (the rest of every address is an immediate)
    const int k_lane = (r32 & 15) * PF_KP + (r32 >> 4) * 512 + h * 16;
    const int vs = lane & 15, vnh = (lane >> 4) & 1;
    const int v_lane = PF_KB + (4 * h + (vs >> 2)) * PF_VP + 32 * vnh + 8 * (vs & 3);
    float* bc = reinterpret_cast<float*>(bc_lds[wave]);

    uint8_t* const st0 = lds_s0 + g * PF_STAGE;  // this group's stages
    uint8_t* const st1 = lds_s1 + g * PF_STAGE;
    if (j_begin < j_end) issue_tile(j_begin, st0);
    pf_wait_vm0();
    __syncthreads();  // Q rows and the first K/V tile landed
    // Q^T operand: lane l holds token t0 + l%32 (clamped), dims 16ks + 8h .. +7, fp16
    h8 qb[16];
    {
        const uint8_t* qr = q_stage(w) + (r32 & 15) * PF_KP + (r32 >> 4) * 512 + 16 * h;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) qb[ks] = pf_lds_h8(qr + 32 * ks);
    }
    __syncthreads();  // every wave holds its Q (the staging stage takes the next tile's copies)
    // one tile: its K/V are in stage `cur`, the next tile is copied into `nxt` meanwhile
    auto tile_step = [&](int it, const uint8_t* cur, uint8_t* nxt) {
        const int j = j_begin + it;
        if (j < j_end) {
            // the next tile (the last one repeats itself into the free stage: no branch around the copies)
            issue_tile(min(j + 1, j_end - 1), nxt);
            const uint8_t* kl = cur + k_lane;
            const uint8_t* vl = cur + v_lane;
            const int j0 = j * PF_BK;

            // S^T: lane reads tile row l%32, chunk 2ks + h
            f16x s;
#pragma unroll
            for (int r = 0; r < 16; r++) s[r] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 16; ks++) {
                s = mfma32(pf_lds_h8(kl + ks * 32), qb[ks], s);
                // two operand reads, their two MFMAs, then one of the next tile's 8 copies: each copy's issue
                // (tens of cycles of this wave) overlaps MFMAs in flight instead of holding up the first ones
                // (a burst of 8 copies before the S product: prefill_4k 161-171 against 154-160 us)
                if ((ks & 1) == 1) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // 2 DS reads
                if ((ks & 1) == 1) __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // 2 MFMAs
                if ((ks & 1) == 1) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // 1 tile copy
            }

            // the V operands of the first two PV MFMAs are read now, so that their latency hides behind the softmax
            // (the V tile landed with K; 3% fewer cycles per call; three or four such steps spill registers)
            h4 vpre[2][2];
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
                vpre[dt][0] = pf_lds_tr(vl + 64 * dt);
                vpre[dt][1] = pf_lds_tr(vl + 64 * dt + 8 * PF_VP);
            }
            // causal mask on tiles that cross the diagonal; register r holds key j0 + 8(r/4) + 4h + r%4
            if (j0 + PF_BK - 1 > off + t0) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = j0 + 8 * (r >> 2) + 4 * h + (r & 3);
                    s[r] = key <= qpos ? s[r] : -INFINITY;
                }
            }
            float tm = s[0];
#pragma unroll
            for (int r = 1; r < 16; r++) tm = fmaxf(tm, s[r]);
            tm = max_xhalf(tm);
            const float tmax = tm * sc;  // log2 domain
            // Conditional rescale: m_run moves only when the row's tile max exceeds it by more than 8 (log2
            // units); otherwise p = 2^(x - m_run) <= 256 stays well inside fp16 and the final division by l
            // cancels the common factor. Rows with no key yet (m_run = -inf) have O = 0 and just take the max.
            float alpha = 1.0f;
            bool moved = false;
            if (tmax > m_run + 8.0f) {
                moved = m_run != -INFINITY;
                alpha = moved ? __builtin_amdgcn_exp2f(m_run - tmax) : 0.0f;
                m_run = tmax;
            }
            if (__ballot(moved)) {
                if (h == 0) bc[r32] = alpha;
                f4 al[4];
#pragma unroll
                for (int gg = 0; gg < 4; gg++) al[gg] = bc_lds[wave][2 * gg + h];
#pragma unroll
                for (int dt = 0; dt < 8; dt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[dt][r] *= al[r >> 2][r & 3];
            }
            l_run *= alpha;
            const float m_use = m_run == -INFINITY ? 0.0f : m_run;
            h8 pa[2];
#pragma unroll
            for (int r = 0; r < 16; r++) pa[r >> 3][r & 7] = (_Float16)__builtin_amdgcn_exp2f(fmaf(s[r], sc, -m_use));
            const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
            for (int k = 0; k < 2; k++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const h2 pp = {pa[k][2 * e], pa[k][2 * e + 1]};
                    l_run = __builtin_amdgcn_fdot2(pp, one, l_run, false);
                }

            // O += P V over the 32 keys: two 16-key steps; V operand rows 16kk + 8rd + 4h + (l%16)/4
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
#pragma unroll
                for (int dt = 0; dt < 8; dt++) {
                    const int imm0 = kk * 512 + 64 * dt;
                    const bool pre = kk == 0 && dt < 2;
                    const h4 x0 = pre ? vpre[dt & 1][0] : pf_lds_tr(vl + imm0);
                    const h4 x1 = pre ? vpre[dt & 1][1] : pf_lds_tr(vl + imm0 + 8 * PF_VP);
                    const h8 vop = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
                    o[dt] = mfma32(pa[kk], vop, o[dt]);
                }
            }
        }
        pf_wait_vm0();    // next tile has landed in LDS
        __syncthreads();  // ... for every wave, and every wave is done with this one
    };
    // unrolled by two so every copy and every read names its stage object at compile time
    for (int it = 0; it < half; it += 2) {
        tile_step(it, st0, st1);
        if (it + 1 < half) tile_step(it + 1, st1, st0);
    }

    // Merge of the two key-range halves (group order), then 1/l and the gate. Group 0 finishes dims 0..127,
    // group 1 dims 128..255; each hands the other half of its O over through LDS (the K/V stages are free now).
    // The gate rows of the finished half are fetched first (coalesced, 16 bytes per lane: lane l covers row
    // 2i + l/32, dims 4(l%32) .. +3 of the half), so their latency hides behind the merge. The group index is
    // a compile-time constant inside `finish`, so the half of O that is handed over dies at the exchange.
    const float l_tot = sum_xhalf(l_run);
    auto finish = [&](auto G) {
        constexpr int gg_ = decltype(G)::value;
        constexpr int dh = gg_ ? 128 : 0;      // first dim this wave finishes
        constexpr int give = gg_ ? 0 : 4;      // O tiles handed to the other group
        constexpr int keep = gg_ ? 4 : 0;      // O tiles finished here
        f4 gz[16];
        if (a.gate) {
            const float* zp = a.gate + (int64_t)head * a.g_hs + dh + 4 * r32;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int t = min(t0 + 2 * i + h, a.T - 1);
                gz[i] = *reinterpret_cast<const f4*>(zp + (int64_t)t * a.g_ts);
            }
        }
        if (h == 0) {
            ml_lds[gg_][w][0][r32] = m_run;
            ml_lds[gg_][w][1][r32] = l_tot;
        }
        {
            // handed-over half, 16 bytes per lane: element (d, r) at ((4d + r/4) * 64 + lane) * 16 + 4 (r%4)
            f4* xs = reinterpret_cast<f4*>((gg_ ? lds_s1 : lds_s0) + w * PF_XSLOT);
#pragma unroll
            for (int d = 0; d < 4; d++)
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    f4 v;
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = o[give + d][4 * q4 + e];
                    xs[(4 * d + q4) * 64 + lane] = v;
                }
        }
        __syncthreads();
        {
            const float m0 = ml_lds[0][w][0][r32], m1 = ml_lds[1][w][0][r32];
            const float l0 = ml_lds[0][w][1][r32], l1 = ml_lds[1][w][1][r32];
            const float M = fmaxf(m0, m1);
            const float w0 = m0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m0 - M);
            const float w1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - M);
            const float inv = 1.0f / (l0 * w0 + l1 * w1);
            // own group's factor first, then the other group's
            if (h == 0) {
                bc[r32] = (gg_ ? w1 : w0) * inv;
                bc[32 + r32] = (gg_ ? w0 : w1) * inv;
            }
        }
        f4 fo[4], fx[4];
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            fo[q4] = bc_lds[wave][2 * q4 + h];
            fx[q4] = bc_lds[wave][8 + 2 * q4 + h];
        }
        // merged rows of the finished half, in the slot this wave read from (only this wave touches it): 32-dim
        // column block d of the half goes to bytes [4096 d, 4096 (d+1)), the same range its handed-over input
        // occupied, as [32 rows][32 dims]; then read back 16 bytes per lane (row 2i + l/32, dims 4(l%32) .. +3)
        // for coalesced stores
        f4* xr = reinterpret_cast<f4*>((gg_ ? lds_s0 : lds_s1) + w * PF_XSLOT);
        float* yr = reinterpret_cast<float*>(xr);
#pragma unroll
        for (int d = 0; d < 4; d++) {
            f4 oth[4];
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) oth[q4] = xr[(4 * d + q4) * 64 + lane];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float y = o[keep + d][r] * fo[r >> 2][r & 3] + oth[r >> 2][r & 3] * fx[r >> 2][r & 3];
                yr[d * 1024 + (8 * (r >> 2) + 4 * h + (r & 3)) * 32 + r32] = y;
            }
        }
        if (a.signs) {
            // gated rows times the signs go back to the same LDS slot (each lane rewrites what it read), for the
            // rotation below
            const f4 sg = *reinterpret_cast<const f4*>(a.signs + (int64_t)head * D + dh + 4 * r32);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                f4& yl = xr[(r32 >> 3) * 256 + (2 * i + h) * 8 + (r32 & 7)];
                f4 y = yl;
                if (a.gate) {
#pragma unroll
                    for (int e = 0; e < 4; e++) y[e] = gate_mul_fast(y[e], gz[i][e]);
                }
                yl = y * sg;
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = t0 + 2 * i + h;
            f4 y = xr[(r32 >> 3) * 256 + (2 * i + h) * 8 + (r32 & 7)];
            if (t < a.T) {
                if (a.gate) {
#pragma unroll
                    for (int e = 0; e < 4; e++) y[e] = gate_mul_fast(y[e], gz[i][e]);
                }
                // the output streams out non-temporally (about 1% fewer cycles than ordinary stores)
                __builtin_nontemporal_store(y, reinterpret_cast<f4*>(a.out + (int64_t)t * a.o_ts + (int64_t)head * a.o_hs +
                                                                   dh + 4 * r32));
            }
        }
    };
    if (g == 0)
        finish(std::integral_constant<int, 0>{});
    else
        finish(std::integral_constant<int, 1>{});

    if (a.signs) {
        // The block's 32 rows x 2 blocks of 512 (heads 2j, 2j+1 of this kv head) are rotated by one wave each,
        // 8 per wave: row 4 wave + k/2, block k%2. Lane l holds dims 4l .. 4l+3 of heads 2j and 2j+1 (the
        // mapping of rotate_pair_store); dim 4l + c was finished by group l/32: its value sits in that group's
        // slot of that head (group 0: lds_s1, group 1: lds_s0) at float ((dim%128)/32) * 1024 + row * 32 +
        // dim % 32, so a lane's four dims are one 16-byte read.
        __syncthreads();
        const int dd = 4 * (lane & 31);
        const uint8_t* gslot = lane < 32 ? lds_s1 : lds_s0;
#pragma unroll 1
        for (int k = 0; k < 8; k++) {
            const int r = 4 * wave + (k >> 1), j = k & 1, t = t0 + r;
            if (t >= a.T) break;  // rows are in order: the rest are past the end too
            float v[8];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float* slot = reinterpret_cast<const float*>(gslot + (2 * j + i) * PF_XSLOT);
                const f4 x = *reinterpret_cast<const f4*>(slot + (dd >> 5) * 1024 + r * 32 + (dd & 31));
#pragma unroll
                for (int c = 0; c < 4; c++) v[4 * i + c] = x[c];
            }
            fwht512_wave(v, lane);
            float* o = a.out + (int64_t)t * a.o_ts + (int64_t)(kh * 4 + 2 * j) * a.o_hs;
#pragma unroll
            for (int i = 0; i < 2; i++)
                __builtin_nontemporal_store(f4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]} * INV_SQRT512,
                                            reinterpret_cast<f4*>(o + i * a.o_hs + 4 * lane));
        }
    }
}

}  // namespace bn
