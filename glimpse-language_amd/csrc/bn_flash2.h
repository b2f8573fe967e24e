// Causal GQA prefill for long query blocks (T >= 64) on fp16 MFMA, 64 query rows per wave.
//
// Semantics follow attn_split.comp:9-58 + attn_combine.comp:6-21 + gate_rotate.comp:19-22 of the reference:
// row t (position off+t) of head h attends to cache rows [0, off+t+1) of kv head h/4; softmax(q.k/16) v,
// then a * sigmoid(gate). The K/V rows of the call are appended to the cache before this kernel runs.
//
// Decomposition (this kernel's own):
//   Block = 4 waves, one per SIMD. Wave w owns query head 4*kh + w and 64 consecutive tokens (two 32-row MFMA
//   blocks), so the block covers 256 query rows that share every K/V tile staged in LDS. With 64 rows per wave
//   each K or V operand read from LDS feeds two MFMAs, which keeps the LDS traffic at about half of what the
//   MFMA pipe consumes (one ds_read per 2 v_mfma_f32_32x32x16_f16).
//   K/V tiles of 64 keys are copied HBM/L2 -> LDS by global_load_lds (no VGPRs), double-buffered. Rows r and
//   r+32 of a tile share one 1 KB copy instruction; the pairs are padded (K: 16 B, V: 64 B per pair) so that the
//   K operand reads (16 rows x 16 B per 16 lanes) and the transposed V reads (ds_read_b64_tr_b16, 4 rows x 32 B
//   per 16 lanes) fall on distinct banks, and every LDS address is one per-lane base register plus an immediate.
//   Each 64-key tile is processed as two 32-key halves (S^T for 32 keys x 64 rows = 32 registers):
//     S^T = K Q^T on v_mfma_f32_32x32x16_f16 (A = K from LDS, B = Q^T in registers, fp16);
//     softmax in fp32, log2 domain (scores scaled by log2(e)/16), against a per-row reference max that stays
//     fixed unless a row max grows by more than 2^14 (then the block restarts), so the 256 O accumulators are
//     never rescaled inside the loop;
//     O += P V with P taken straight from the S^T registers as the A operand and V from two transposed reads.
//   Causal masking only on tiles that cross the diagonal; tiles past it are not visited.
//   Block order: longest q-tiles first, each kv head pinned to a fixed set of XCDs. When the q-tiles alone cannot
//   fill the GPU the key range of a q-tile is split; each split writes (m, l, acc) per row and
//   flash2_combine_kernel merges them in split order.
#pragma once
#include "bn_device.h"

namespace bn {

constexpr int F2_BQ = 64;                       // tokens per q-tile (per wave)
constexpr int F2_BK = 64;                       // keys per K/V tile
constexpr int F2_ROWS = 4 * F2_BQ;              // query rows per block
constexpr int F2_KP = 1040;                     // bytes per K row pair (rows r, r+32) in LDS
constexpr int F2_VP = 1088;                     // bytes per V row pair
constexpr int F2_KB = 32 * F2_KP;               // K stage bytes
constexpr int F2_STAGE = F2_KB + 32 * F2_VP;    // K + V stage bytes (68,096)

struct Flash2Args {
    const float* q;          // element t*q_ts + h*q_hs + d (fp32) ...
    const uint16_t* q16;     // ... or fp16 bits when non-null
    int64_t q_ts, q_hs;
    const uint16_t* kc;      // fp16 [rows][KV][256]
    const uint16_t* vc;
    const float* gate;       // element t*g_ts + h*g_hs + d, or null
    int64_t g_ts, g_hs;
    float* out;              // element t*o_ts + h*o_hs + d
    int64_t o_ts, o_hs;
    float* part_acc;         // [KV][ntq][max_splits][256 rows][256]
    float* part_ml;          // [KV][ntq][max_splits][256 rows][2]: m (log2 domain), l
    int T, off, KV, ntq;
    int ct;                  // K tiles per split
    int max_splits;
};

typedef short f2_s4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f2_s4v f2_lds_s4_t;
typedef __attribute__((address_space(3))) void f2_lds_void_t;

__device__ __forceinline__ h8 f2_lds_h8(const uint8_t* p) { return *reinterpret_cast<const h8*>(p); }
__device__ __forceinline__ h4 f2_lds_tr(const uint8_t* p) {
    return __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((f2_lds_s4_t*)(p)));
}
__device__ __forceinline__ void f2_wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// S^T MFMAs with their accumulator in VGPRs. The O accumulators fill all 256 AGPRs, and the builtin would give
// every MFMA an AGPR accumulator; the asm form keeps the 32 S^T registers in VGPRs. The chain needs no wait
// states between links (the accumulator is exactly the previous result); f2_s_ready() covers the wait before
// VALU instructions read the result (at most 20 wait states for an XDL op on gfx950).
__device__ __forceinline__ f16x f2_mfma_s0(h8 a, h8 b) {
    f16x d;
    asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
__device__ __forceinline__ void f2_mfma_s(f16x& c, h8 a, h8 b) {
    asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void f2_s_ready(f16x& x, f16x& y) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(x), "+v"(y));
}

// exp2 on v_exp_f32 directly (results below 2^-126 flush to zero, which the softmax sums do not notice)
__device__ __forceinline__ float f2_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__global__ __launch_bounds__(256) void flash2_kernel(Flash2Args a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * F2_STAGE];
    __shared__ f4 bc_lds[4][16];  // per wave: 64 floats broadcast in row order (row totals l)

    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, r32 = lane & 31;
    const int KV = a.KV, ntq = a.ntq;

    // block -> (kv head, q-tile, split)
    int kh, qt, s;
    {
        const int b = blockIdx.x;
        if (a.max_splits == 1) {
            const int nb = KV * ntq;
            int idx;
            if (8 % KV == 0 && nb % 8 == 0) {
                // XCD x (= b % 8) serves kv head x % KV; longest q-tiles (highest index) first
                const int xcd = b & 7, reps = 8 / KV;
                kh = xcd % KV;
                idx = (b >> 3) * reps + xcd / KV;
            } else {
                kh = b % KV;
                idx = b / KV;
            }
            qt = ntq - 1 - idx;
            s = 0;
        } else {
            s = b % a.max_splits;
            qt = (b / a.max_splits) % ntq;
            kh = b / (a.max_splits * ntq);
        }
    }
    const int t0 = qt * F2_BQ;
    const int t_last = min(a.T, t0 + F2_BQ) - 1;
    const int nk = a.off + a.T;                          // cache rows that exist
    const int kt_all = (a.off + t_last + 1 + F2_BK - 1) / F2_BK;
    const int kt0 = s * a.ct;
    if (kt0 >= kt_all) return;
    const int kt1 = min(kt_all, kt0 + a.ct);
    const int64_t kvd = (int64_t)KV * D;
    const uint16_t* kb = a.kc + (int64_t)kh * D;
    const uint16_t* vb = a.vc + (int64_t)kh * D;
    const int head = kh * 4 + w;

    // Q^T operands: row block b, lane l holds token t0 + 32b + l%32 (clamped), dims 16ks + 8h .. +7, fp16
    h8 qb[2][16];
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const int tl = min(t0 + 32 * b + r32, a.T - 1);
        if (a.q16) {
            const uint16_t* qr = a.q16 + (int64_t)tl * a.q_ts + (int64_t)head * a.q_hs + 8 * h;
#pragma unroll
            for (int ks = 0; ks < 16; ks++) qb[b][ks] = ld_h8(qr + ks * 16);
        } else {
            const float* qr = a.q + (int64_t)tl * a.q_ts + (int64_t)head * a.q_hs + 8 * h;
#pragma unroll
            for (int ks = 0; ks < 16; ks++) qb[b][ks] = ld_f32x8_as_h8(qr + ks * 16);
        }
    }

    // Tile copy: wave w moves row pairs 8w .. 8w+7 of K and of V; lane l of an instruction loads row
    // p + 32*(l/32), 16-byte chunk l%32, into LDS pair p at byte 16*l. Rows past the cache are clamped to its
    // last row (masked, or never read).
    auto issue_tile = [&](int kt, int buf) {
        const int j0 = kt * F2_BK;
        const int lim = nk - 1 - j0;                       // last valid row of this tile
        const char* kt_base = reinterpret_cast<const char*>(kb + (int64_t)j0 * kvd);  // wave-uniform
        const char* vt_base = reinterpret_cast<const char*>(vb + (int64_t)j0 * kvd);
        uint8_t* st = lds + buf * F2_STAGE;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int p = 8 * w + i;
            // byte offset inside this tile's 64 rows: uniform base + 32-bit lane offset (saddr form)
            const uint32_t g = (uint32_t)(min(p + 32 * h, lim) * (int)kvd + r32 * 8) * 2u;
            __builtin_amdgcn_global_load_lds(kt_base + g, (f2_lds_void_t*)(st + p * F2_KP), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vt_base + g, (f2_lds_void_t*)(st + F2_KB + p * F2_VP), 16, 0, 0);
        }
    };

    // Softmax reference: row r's probabilities are p = 2^(x - m_ref[r]) with m_ref fixed between restarts, so
    // the O accumulators are never rescaled in the loop. m_ref is set by the first tile that has a key for the
    // row (O is still zero then). If a later tile's row max exceeds m_ref by more than F2_GROW (p would leave the
    // fp16 range), the whole block restarts from its first tile with m_ref = the largest max seen so far; the
    // tile that triggered it is discarded (its p are clamped so nothing overflows meanwhile). Restarts need a
    // row max that grows by more than 2^14 after its first tile, which is rare; they always terminate, because
    // after a restart every tile seen so far is within range.
    constexpr float F2_GROW = 14.0f;
    __shared__ int restart_lds;
    if (tid == 0) restart_lds = 0;

    f16x o[2][8];
    float m_ref[2] = {-INFINITY, -INFINITY}, m_seen[2] = {-INFINITY, -INFINITY}, l_run[2];
    const float sc = QK_SCALE * LOG2E;

    // per-lane LDS bases (the rest of every address is an immediate)
    const int k_lane = r32 * F2_KP + h * 16;
    const int vs = lane & 15, vnh = (lane >> 4) & 1;
    const int v_lane = F2_KB + (4 * h + (vs >> 2)) * F2_VP + 32 * vnh + 8 * (vs & 3);

    issue_tile(kt0, 0);
    f2_wait_vm0();
    __syncthreads();
    int kt = kt0;
restart:
#pragma unroll
    for (int b = 0; b < 2; b++) {
        l_run[b] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[b][dt][r] = 0.0f;
    }
    for (; kt < kt1; kt++) {
        const int buf = (kt - kt0) & 1;
        if (kt + 1 < kt1) issue_tile(kt + 1, buf ^ 1);
        const uint8_t* kl = lds + buf * F2_STAGE + k_lane;
        const uint8_t* vl = lds + buf * F2_STAGE + v_lane;
        const int j0 = kt * F2_BK;
        const bool diag = j0 + F2_BK - 1 > a.off + t0;
        bool grow = false;

#pragma unroll 1
        for (int k2 = 0; k2 < 2; k2++) {
            // S^T for keys 32k2 .. 32k2+31 of the tile: lane reads key row 32k2 + l%32, dims 16ks + 8h
            f16x st[2];
            {
                const h8 kop = f2_lds_h8(kl + k2 * 512);
                st[0] = f2_mfma_s0(kop, qb[0][0]);
                st[1] = f2_mfma_s0(kop, qb[1][0]);
            }
#pragma unroll
            for (int ks = 1; ks < 16; ks++) {
                const h8 kop = f2_lds_h8(kl + k2 * 512 + ks * 32);
                f2_mfma_s(st[0], kop, qb[0][ks]);
                f2_mfma_s(st[1], kop, qb[1][ks]);
            }
            f2_s_ready(st[0], st[1]);
            // probabilities of both row blocks (lane row = token t0 + 32b + l%32)
            h8 pa[2][2];
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const int qpos = a.off + t0 + 32 * b + r32;
                float x[16];
                float tmax = -INFINITY;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    x[r] = st[b][r] * sc;
                    if (diag) {
                        const int j = j0 + 32 * k2 + 8 * (r >> 2) + 4 * h + (r & 3);
                        x[r] = j <= qpos ? x[r] : -INFINITY;
                    }
                    tmax = fmaxf(tmax, x[r]);
                }
                tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
                m_seen[b] = fmaxf(m_seen[b], tmax);
                if (m_ref[b] == -INFINITY) m_ref[b] = tmax;  // first keys of this row: O is still zero
                grow |= tmax > m_ref[b] + F2_GROW;
                const float m_use = m_ref[b] == -INFINITY ? 0.0f : m_ref[b];
                float psum = 0.0f;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float p = f2_exp2(fminf(x[r] - m_use, 15.0f));
                    psum += p;
                    pa[b][r >> 3][r & 7] = (_Float16)p;
                }
                l_run[b] += psum;
            }
            // O += P V over the 32 keys: two 16-key steps; V operand rows 32k2 + 16kk + 8rd + 4h + (l%16)/4
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
#pragma unroll
                for (int dt = 0; dt < 8; dt++) {
                    const int imm0 = (16 * kk) * F2_VP + k2 * 512 + 64 * dt;
                    const h4 x0 = f2_lds_tr(vl + imm0);
                    const h4 x1 = f2_lds_tr(vl + imm0 + 8 * F2_VP);
                    const h8 vop = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                    o[0][dt] = mfma32(pa[0][kk], vop, o[0][dt]);
                    o[1][dt] = mfma32(pa[1][kk], vop, o[1][dt]);
                }
            }
        }
        if (__ballot(grow)) restart_lds = 1;  // benign race: every writer stores 1

        f2_wait_vm0();    // next tile has landed in LDS
        __syncthreads();  // ... for every wave, and every wave is done with this one
        if (restart_lds) {
            __syncthreads();  // every wave has read the flag
            if (tid == 0) restart_lds = 0;
            m_ref[0] = m_seen[0];
            m_ref[1] = m_seen[1];
            kt = kt0;
            asm volatile("" : "+s"(kt));  // opaque: keeps this rare path's copy addresses out of the loop preheader
            issue_tile(kt, 0);
            f2_wait_vm0();
            __syncthreads();
            goto restart;
        }
    }

    // row totals (both lane halves hold the same row), broadcast to the O register layout
    float lv[2][16];
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const float l_tot = l_run[b] + __shfl_xor(l_run[b], 32);
        float* bc = reinterpret_cast<float*>(bc_lds[w]);
        if (h == 0) bc[32 * b + r32] = l_tot;
    }
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const f4 x = bc_lds[w][8 * b + 2 * g + h];
#pragma unroll
            for (int e = 0; e < 4; e++) lv[b][4 * g + e] = x[e];
        }

    if (a.max_splits == 1) {
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int t = t0 + 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
                if (t >= a.T) continue;
                float* op = a.out + (int64_t)t * a.o_ts + (int64_t)head * a.o_hs + r32;
                const float* zp = a.gate ? a.gate + (int64_t)t * a.g_ts + (int64_t)head * a.g_hs + r32 : nullptr;
                const float inv = __builtin_amdgcn_rcpf(lv[b][r]);
#pragma unroll
                for (int dt = 0; dt < 8; dt++) {
                    float y = o[b][dt][r] * inv;
                    if (zp) y = gate_mul_fast(y, zp[32 * dt]);
                    op[32 * dt] = y;
                }
            }
        return;
    }
    // split partials: unnormalised rows, m and l per row
    const int64_t prow = (((int64_t)kh * ntq + qt) * a.max_splits + s) * F2_ROWS + w * F2_BQ;
#pragma unroll
    for (int b = 0; b < 2; b++) {
        if (h == 0) {
            a.part_ml[(prow + 32 * b + r32) * 2] = m_ref[b];
            a.part_ml[(prow + 32 * b + r32) * 2 + 1] = l_run[b] + __shfl_xor(l_run[b], 32);
        }
    }
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int rr = 32 * b + 8 * (r >> 2) + 4 * h + (r & 3);
            float* pp = a.part_acc + (prow + rr) * D + r32;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) pp[32 * dt] = o[b][dt][r];
        }
}

// Merge of the key splits of one (token, head) row in split order (attn_combine.comp:10-20), then the gate.
// Grid (T, H) x 64 threads; thread: dims 4*lane .. +3.
__global__ __launch_bounds__(64) void flash2_combine_kernel(Flash2Args a) {
    const int t = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
    const int kh = head >> 2, w = head & 3, qt = t / F2_BQ;
    const int t_last = min(a.T, qt * F2_BQ + F2_BQ) - 1;
    const int kt_all = (a.off + t_last + 1 + F2_BK - 1) / F2_BK;
    const int ns = (kt_all + a.ct - 1) / a.ct;
    const int64_t row0 = (((int64_t)kh * a.ntq + qt) * a.max_splits) * F2_ROWS + w * F2_BQ + (t % F2_BQ);
    float M = -INFINITY;
    for (int sp = 0; sp < ns; sp++) M = fmaxf(M, a.part_ml[(row0 + (int64_t)sp * F2_ROWS) * 2]);
    float L = 0.0f;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp = 0; sp < ns; sp++) {
        const int64_t rw = row0 + (int64_t)sp * F2_ROWS;
        const float m = a.part_ml[rw * 2];
        if (m == -INFINITY) continue;
        const float wgt = exp2f(m - M);
        L = fmaf(a.part_ml[rw * 2 + 1], wgt, L);
        const f4 v = *reinterpret_cast<const f4*>(a.part_acc + rw * D + 4 * lane);
#pragma unroll
        for (int e = 0; e < 4; e++) acc[e] = fmaf(v[e], wgt, acc[e]);
    }
    const float* zp = a.gate ? a.gate + (int64_t)t * a.g_ts + (int64_t)head * a.g_hs + 4 * lane : nullptr;
    f4 y;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        y[e] = acc[e] / L;
        if (zp) y[e] = gate_mul(y[e], zp[e]);
    }
    *reinterpret_cast<f4*>(a.out + (int64_t)t * a.o_ts + (int64_t)head * a.o_hs + 4 * lane) = y;
}

}  // namespace bn
