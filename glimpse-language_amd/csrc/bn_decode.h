// Split-KV decode attention (one query token per sequence) over an fp16 KV cache.
//
// Semantics follow attn_split.comp:9-58 + attn_combine.comp:6-21 + gate_rotate.comp:19-22 of the reference
// (query row of head h attends to cache rows [0, L) of kv head h/4, softmax(q.k / 16), gate a*sigmoid(z));
// the decomposition is this kernel's own:
//   grid (split, kv head, sequence) x one wave. A split covers `chunk` consecutive keys of one kv head and
//   serves the 4 query heads that share it, so every K/V byte is read once.
//   QK^T: v_mfma_f32_16x16x32_f16 computes S^T = K Q^T over 16-key tiles. The A operand is the K tile read
//   straight from HBM in MFMA layout (lane: key l%16, 8 dims per k-step); the B operand holds the 4 heads'
//   query rows as an fp16 hi/lo pair (columns h and h+4, repeated in 8..15), so hi + lo carries the fp32
//   query and the scores are fp32-accurate at no extra MFMA cost.
//   Softmax: online, in the log2 domain (q pre-scaled by log2 e), fp32.
//   PV: fp32 FMAs on the VALU; each lane owns 8 dims of every other key and the 4 heads.
//   Combine: a sequence that fits one split is finished (divided and gated) by its split. Otherwise each
//   split writes (m, l, acc[256]) per head to the workspace and decode_combine_kernel, launched next on the
//   same stream, merges them in split order and gates. The kernel boundary makes the partials visible
//   across the XCDs' separate L2s; a device-scope fence per block (an L2 write-back plus invalidate on
//   gfx950) would cost far more. The merge order is fixed, so results do not depend on scheduling.
//   Append: when k_new/v_new are given, the new row (last key of the sequence) is taken from them, rounded
//   to fp16, used for the score and the PV product, and stored into the cache by the same split.
#pragma once
#include "bn_device.h"

namespace bn {

constexpr int DEC_PART = 8 + 4 * D;  // per (sequence, kv head, split): m[4], l[4], acc[4][256] (floats)

struct DecodeArgs {
    const float* q;      // element seq*q_ss + head*q_hs + d (fp32) ...
    const uint16_t* q16; // ... or fp16 bits when non-null
    int64_t q_ss, q_hs;
    const float* k_new;  // element seq*kn_ss + kh*256 + d, or null
    const float* v_new;
    int64_t kn_ss;
    uint16_t* kc;        // fp16 rows [row][KV][256]
    uint16_t* vc;
    const int64_t* kv_off;  // device: first cache row of each sequence (null: row0 + seq*row_step)
    const int32_t* kv_len;  // device: keys of each sequence (null: len0 + seq*len_step)
    int64_t row0, row_step;
    int32_t len0, len_step;
    const float* gate;   // element seq*g_ss + head*g_hs + d, or null
    int64_t g_ss, g_hs;
    float* out;          // element seq*o_ss + head*o_hs + d
    int64_t o_ss, o_hs;
    float* part;         // [nseq][KV][max_splits][DEC_PART]
    int KV, chunk, max_splits, max_len;
};

__global__ __launch_bounds__(64) void decode_split_kernel(DecodeArgs a) {
    __shared__ f4 p_lds[16];   // p[key in tile][head]
    __shared__ f4 al_lds;      // per-head rescale of the running accumulators
    __shared__ f4 ml_lds[2];   // final m, l per head

    const int s = blockIdx.x, kh = blockIdx.y, seq = blockIdx.z;
    const int lane = threadIdx.x;
    // keys of this sequence; device-supplied lengths are clamped to the launch bound
    const int L = min(a.kv_len ? a.kv_len[seq] : a.len0 + seq * a.len_step, a.max_len);
    const int64_t row0 = a.kv_off ? a.kv_off[seq] : a.row0 + (int64_t)seq * a.row_step;
    const int ns = L > 0 ? (L + a.chunk - 1) / a.chunk : 0;
    if (s >= ns) return;
    const int j0 = s * a.chunk;
    const int j1 = min(L, j0 + a.chunk);
    const bool has_new = a.k_new != nullptr && j1 == L;  // this split owns the appended row L-1
    const int tl = j0 + (j1 - j0 - 1) / 16 * 16;          // first key of the split's last (maybe partial) tile
    const int64_t kvd = (int64_t)a.KV * D;
    const uint16_t* kb = a.kc + (row0 * a.KV + kh) * D;
    const uint16_t* vb = a.vc + (row0 * a.KV + kh) * D;

    const int c = lane & 15, g = lane >> 4;       // MFMA column / k-group of this lane
    const int pvr = lane >> 5, pvd = (lane & 31) * 8;  // PV layout: key parity, first dim

    // B operand: Q^T, column c = head (c&3), hi part for (c&4)==0 else lo part, k-step ks covers
    // dims ks*32 + g*8 .. +7.
    h8 qb[8];
    {
        const int64_t qo = seq * a.q_ss + (int64_t)(kh * 4 + (c & 3)) * a.q_hs + g * 8;
        const bool lo = (c & 4) != 0;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            float x[8];
            if (a.q16) {
                const h8 v = ld_h8(a.q16 + qo + ks * 32);
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = (float)v[e];
            } else {
                const f4 u = *reinterpret_cast<const f4*>(a.q + qo + ks * 32);
                const f4 v = *reinterpret_cast<const f4*>(a.q + qo + ks * 32 + 4);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    x[e] = u[e];
                    x[e + 4] = v[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float y = x[e] * LOG2E;
                const _Float16 hi = (_Float16)y;
                qb[ks][e] = lo ? (_Float16)(y - (float)hi) : hi;
            }
        }
    }

    float m_run = -INFINITY, l_run = 0.0f;
    float acc[4][8];
#pragma unroll
    for (int h = 0; h < 4; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;

    auto tile = [&](const h8* kt, const h8* vt, int jt, int jlim) {
        f4 sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 8; ks++) sacc = mfma16(kt[ks], qb[ks], sacc);
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v = (sacc[r] + __shfl_xor(sacc[r], 4)) * QK_SCALE;
            sc[r] = (jt + 4 * g + r < jlim) ? v : -INFINITY;
        }
        float tm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        tm = fmaxf(tm, __shfl_xor(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        const float m_new = fmaxf(m_run, tm);
        const float alpha = exp2f(m_run - m_new);
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; r++) p[r] = exp2f(sc[r] - m_new);
        l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        m_run = m_new;
        if (c < 4) {
#pragma unroll
            for (int r = 0; r < 4; r++) p_lds[4 * g + r][c] = p[r];
            if (g == 0) al_lds[c] = alpha;
        }
        __syncthreads();
        const f4 al = al_lds;
#pragma unroll
        for (int h = 0; h < 4; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[h][e] *= al[h];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f4 pv = p_lds[2 * i + pvr];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float v = (float)vt[i][e];
#pragma unroll
                for (int h = 0; h < 4; h++) acc[h][e] = fmaf(pv[h], v, acc[h][e]);
            }
        }
        __syncthreads();
    };

    // rows past the split end are clamped to its last row (in bounds; their scores are masked)
    auto load_k = [&](int jt, h8* kt) {
        const int r = min(jt + c, j1 - 1);
        const uint16_t* p = kb + (int64_t)r * kvd + g * 8;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) kt[ks] = ld_h8_nt(p + ks * 32);
    };
    auto load_v = [&](int jt, h8* vt) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int r = min(jt + 2 * i + pvr, j1 - 1);
            vt[i] = ld_h8_nt(vb + (int64_t)r * kvd + pvd);
        }
    };

    // full tiles [j0, tl) with the next tile's loads in flight, then the last tile [tl, j1)
    h8 kt[8], vt[8];
    load_k(j0, kt);
    load_v(j0, vt);
    for (int jt = j0; jt < tl; jt += 16) {
        h8 kn[8], vn[8];
        load_k(jt + 16, kn);
        load_v(jt + 16, vn);
        tile(kt, vt, jt, j1);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            kt[i] = kn[i];
            vt[i] = vn[i];
        }
    }
    if (has_new) {
        // row L-1 of the last tile comes from k_new / v_new (fp16, nearest even) and is stored to the cache,
        // so a call that appends and one that finds the row cached produce the same bits
        const int rn = L - 1 - tl;  // tile row of the new key
        const float* kn = a.k_new + seq * a.kn_ss + kh * D;
        const float* vn = a.v_new + seq * a.kn_ss + kh * D;
        uint16_t* kdst = a.kc + ((row0 + L - 1) * a.KV + kh) * D;
        uint16_t* vdst = a.vc + ((row0 + L - 1) * a.KV + kh) * D;
        if (c == rn) {
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                kt[ks] = ld_f32x8_as_h8(kn + ks * 32 + g * 8);
                st_h8(kdst + ks * 32 + g * 8, kt[ks]);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (2 * i + pvr == rn) {
                vt[i] = ld_f32x8_as_h8(vn + pvd);
                st_h8(vdst + pvd, vt[i]);
            }
        }
    }
    tile(kt, vt, tl, j1);

    // totals over the lanes holding the same head / dims
    float l_tot = l_run + __shfl_xor(l_run, 16);
    l_tot += __shfl_xor(l_tot, 32);
#pragma unroll
    for (int h = 0; h < 4; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[h][e] += __shfl_xor(acc[h][e], 32);
    if (lane < 4) {
        ml_lds[0][lane] = m_run;
        ml_lds[1][lane] = l_tot;
    }
    __syncthreads();

    if (ns == 1) {
        if (lane < 32) {
            const f4 lsum = ml_lds[1];
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const int head = kh * 4 + h;
                float* o = a.out + seq * a.o_ss + head * a.o_hs + pvd;
                const float* z = a.gate ? a.gate + seq * a.g_ss + head * a.g_hs + pvd : nullptr;
                float y[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    y[e] = acc[h][e] / lsum[h];
                    if (z) y[e] = gate_mul(y[e], z[e]);
                }
                *reinterpret_cast<f4*>(o) = f4{y[0], y[1], y[2], y[3]};
                *reinterpret_cast<f4*>(o + 4) = f4{y[4], y[5], y[6], y[7]};
            }
        }
        return;
    }

    float* pp = a.part + (((int64_t)seq * a.KV + kh) * a.max_splits + s) * DEC_PART;
    if (lane < 4) {
        pp[lane] = ml_lds[0][lane];
        pp[4 + lane] = ml_lds[1][lane];
    }
    if (lane < 32) {
#pragma unroll
        for (int h = 0; h < 4; h++) {
            float* d = pp + 8 + h * D + pvd;
            *reinterpret_cast<f4*>(d) = f4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
            *reinterpret_cast<f4*>(d + 4) = f4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
        }
    }
}

// Merge of the split partials of one (sequence, kv head): M = max m_s, L = sum l_s 2^(m_s - M),
// out = (sum acc_s 2^(m_s - M)) / L, in split order (attn_combine.comp:10-20), then the gate.
// Runs as its own launch after decode_split_kernel, so the partials are visible without device-wide fences.
// Block = one wave per (head, kv head, sequence); lane: dims 4*lane .. +3.
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeArgs a) {
    const int h = blockIdx.x, kh = blockIdx.y, seq = blockIdx.z;
    const int lane = threadIdx.x, d0 = lane * 4;
    const int L = min(a.kv_len ? a.kv_len[seq] : a.len0 + seq * a.len_step, a.max_len);
    const int ns = L > 0 ? (L + a.chunk - 1) / a.chunk : 0;
    if (ns <= 1) return;  // written by the split kernel
    const float* pb = a.part + ((int64_t)seq * a.KV + kh) * a.max_splits * DEC_PART;
    float M = -INFINITY;
    for (int sp = lane; sp < ns; sp += 64) M = fmaxf(M, pb[(int64_t)sp * DEC_PART + h]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) M = fmaxf(M, __shfl_xor(M, m));
    float Ls = 0.0f;
    f4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
    for (int sp = 0; sp < ns; sp++) {
        const float* ps = pb + (int64_t)sp * DEC_PART;
        const float w = exp2f(ps[h] - M);
        Ls = fmaf(ps[4 + h], w, Ls);
        const f4 v = *reinterpret_cast<const f4*>(ps + 8 + h * D + d0);
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = fmaf(v[e], w, o[e]);
    }
    const int head = kh * 4 + h;
    const float* z = a.gate ? a.gate + seq * a.g_ss + head * a.g_hs + d0 : nullptr;
    f4 y;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        y[e] = o[e] / Ls;
        if (z) y[e] = gate_mul(y[e], z[e]);
    }
    *reinterpret_cast<f4*>(a.out + seq * a.o_ss + head * a.o_hs + d0) = y;
}

}  // namespace bn
