// Speculative verify on fp16 MFMA: 2..16 draft rows of one sequence against the cache, every K/V row read once
// for every 8 rows.
//
// Semantics follow attn_split.comp:9-58 + attn_combine.comp:6-21 of the reference: row t (position off+t) of head
// h attends to cache rows [0, off+t+1) of kv head h/4 (causal among the drafts), softmax(q.k/16) v. The K/V rows
// of the call are either in the cache already or given as k_new / v_new: then the wave whose tiles hold them rounds
// them to fp16 and stores them into the cache before its tile copies (no separate append launch). The gate and the
// rotation are decode_combine_kernel's.
//
// Decomposition (this kernel's own):
//   The 4 query heads of a kv head times 8 rows are 32 query rows: one MFMA column tile. Block (split s, kv head
//   kh, row group z) takes rows 8 z .. 8 z + 7 (the reference verifies up to 16 rows: two row groups, each reading
//   the split's K/V rows once); column c = 8 hq + t' holds row 8 z + t' of head 4 kh + hq (columns past the last
//   row repeat it and are dropped). The block covers keys [s chunk, (s+1) chunk) for all 32 columns; its W waves
//   take contiguous runs of the split's 32-key tiles, each wave with its own K/V stage in LDS (the tile layout of
//   prefill_kernel: rows p and p+16 share one 1 KB global_load_lds copy, padded so the operand reads are
//   conflict-free).
//   S^T = K Q^T on v_mfma_f32_32x32x16_f16 (Q^T in registers as fp16; an fp32 q is carried as an fp16 hi/lo
//   pair, hi = fp16(q), lo = fp16(q - hi), both multiplied into the same accumulator, so its scores keep about
//   22 of q's 24 bits at any score scale), online softmax in fp32 in the log2 domain (the running max moves only when a column's max grows by more than 2^8), O += P V with P from the
//   S^T registers and V from ds_read_b64_tr_b16 reads, as in prefill_kernel.
//   The block merges its W waves in wave order through LDS and writes one partial record (m, l, acc) per row and
//   split in decode_combine_kernel's layout (m in the log2 domain, slot 8 (t + T (s / 8)) + s % 8); the combine
//   merges every row's splits in split order, so results are reproducible bit for bit.
#pragma once
#include "bn_decode.h"
#include "bn_prefill.h"

namespace bn {

struct VerifyArgs {
    const float* q;          // element t*q_ts + h*q_hs + d (fp32) ...
    const uint16_t* q16;     // ... or fp16 bits when non-null
    int64_t q_ts, q_hs;
    uint16_t* kc;            // fp16 [rows][KV][256]
    uint16_t* vc;
    const float* k_new;      // the call's rows [T][KV][256] fp32, appended by the kernel, or null (already in the
    const float* v_new;      // cache)
    float* part;             // [KV][units][DEC_PART]
    const uint32_t* dyn;     // device offset (graph replay) or null; off is then its upper bound
    int T, off, KV, chunk, units;
};

constexpr int VF_OP = 1040;  // row pitch (bytes) of a wave's O rows in LDS at the merge

// HILO: q is fp32 (a.q), multiplied as hi + lo; otherwise q is fp16 bits (a.q16)
template <int W, bool HILO>
__global__ __launch_bounds__(64 * W) void verify_kernel(VerifyArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[W * PF_STAGE];
    __shared__ float ml_lds[W][2][32];  // per wave: m, l of each column

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, r32 = lane & 31;
    // every argument word the block needs is requested at entry, in one round trip
    asm volatile("" ::"s"(a.q), "s"(a.q16), "s"(a.q_ts), "s"(a.q_hs), "s"(a.kc), "s"(a.vc), "s"(a.part), "s"(a.dyn),
                 "s"(a.T), "s"(a.off), "s"(a.KV), "s"(a.chunk), "s"(a.units));
    const int s = blockIdx.x, kh = blockIdx.y, KV = a.KV, T = a.T;
    const int off = call_off(a.dyn, a.off);
    const int nk = off + T;                              // cache rows that exist
    const int k0 = s * a.chunk;
    const int k1 = min(k0 + a.chunk, nk);
    const int nt = (k1 - k0 + PF_BK - 1) / PF_BK;        // the split's 32-key tiles
    const int j_begin = w * nt / W, j_end = (w + 1) * nt / W;
    const int64_t kvd = (int64_t)KV * D;
    const uint16_t* kb = a.kc + (int64_t)kh * D;
    const uint16_t* vb = a.vc + (int64_t)kh * D;
    uint8_t* const st = lds + w * PF_STAGE;

    // this lane's column: row t of head 4 kh + hq (the block's rows rb .. rb + 7); its keys are <= qpos
    const int rb = 8 * (int)blockIdx.z;
    // a split that starts past the row group's last position holds no key of its rows (nor a new row: the last row
    // group, which covers every split that holds one, appends those)
    if (k0 > off + min(rb + 7, T - 1)) return;
    const int hq = r32 >> 3, t = min(rb + (r32 & 7), T - 1);
    const int qpos = off + t;

    // Tile copies into this wave's stage, K and V separately: instruction i moves row pair i (rows i, i+16); lane l
    // loads row i + 16 (l/32), 16-byte chunk l%32, into LDS pair i at byte 16 l. Rows past the cache's last row are
    // clamped to it (their scores are masked: every column's qpos < nk). K of tile j + 1 is copied once the S
    // product of tile j has read K, V of tile j + 1 once the PV product has read V, so each copy runs under the other
    // half's work (16 copies each; the waits below count them).
    const uint32_t lane_go = (uint32_t)(16 * h * (int)kvd + r32 * 8) * 2u;
    auto issue_half = [&](int j, const uint16_t* base, int lds_off, int pitch) {
        const int j0 = k0 + j * PF_BK;
        const char* src = reinterpret_cast<const char*>(base + (int64_t)j0 * kvd);
        if (j0 + PF_BK <= nk) {
#pragma unroll
            for (int i = 0; i < 16; i++) pf_copy16(src + i * kvd * 2 + lane_go, st + lds_off + i * pitch);
        } else {
            const int lim = nk - 1 - j0;  // last valid row of this tile
#pragma unroll
            for (int i = 0; i < 16; i++)
                pf_copy16(src + (uint32_t)(min(i + 16 * h, lim) * (int)kvd + r32 * 8) * 2u, st + lds_off + i * pitch);
        }
    };
    auto issue_k = [&](int j) { issue_half(j, kb, 0, PF_KP); };
    auto issue_v = [&](int j) { issue_half(j, vb, PF_KB, PF_VP); };

    f16x o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float sc = QK_SCALE * LOG2E;
    const int k_lane = (r32 & 15) * PF_KP + (r32 >> 4) * 512 + h * 16;
    const int vs = lane & 15, vnh = (lane >> 4) & 1;
    const int v_lane = PF_KB + (4 * h + (vs >> 2)) * PF_VP + 32 * vnh + 8 * (vs & 3);
    __shared__ f4 bc_lds[W][16];
    float* bc = reinterpret_cast<float*>(bc_lds[w]);

    // The call's new rows [off, off + T) that fall in this wave's tiles go to the cache first (fp16, nearest even),
    // before the wave's copies read them: the tiles partition the keys among the waves and splits, and the blocks of
    // the other row group write the same bytes to the same rows before reading them.
    if (a.k_new && !dyn_over(a.dyn, a.off)) {  // past the bound nothing is appended (the flag is set)
        const int r0 = max(off, k0 + j_begin * PF_BK), r1 = min(nk, k0 + j_end * PF_BK);
        // up to 16 rows, 8 at a time
        for (int rr = r0; rr < r1; rr += 8) {
            f4 kn[8], vn[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (rr + i < r1) {
                    const int64_t src = (int64_t)(rr + i - off) * kvd + (int64_t)kh * D + 4 * lane;
                    kn[i] = *reinterpret_cast<const f4*>(a.k_new + src);
                    vn[i] = *reinterpret_cast<const f4*>(a.v_new + src);
                }
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (rr + i < r1) {
                    const int64_t dst = (int64_t)(rr + i) * kvd + (int64_t)kh * D + 4 * lane;
                    const h4 kh4 = {(_Float16)kn[i][0], (_Float16)kn[i][1], (_Float16)kn[i][2], (_Float16)kn[i][3]};
                    const h4 vh4 = {(_Float16)vn[i][0], (_Float16)vn[i][1], (_Float16)vn[i][2], (_Float16)vn[i][3]};
                    *reinterpret_cast<h4*>(a.kc + dst) = kh4;
                    *reinterpret_cast<h4*>(a.vc + dst) = vh4;
                }
        }
        if (r0 < r1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the rows are in L2 before the copies read them
    }
    // the first tile's copies are in flight while the q rows load
    if (j_begin < j_end) {
        issue_k(j_begin);
        issue_v(j_begin);
    }
    // Q^T operand: lane holds column r32, dims 16 ks + 8 h .. +7, fp16 (hi and lo parts for an fp32 q)
    h8 qb[16], ql[HILO ? 16 : 1];
    if constexpr (HILO) {
        const float* qr = a.q + (int64_t)t * a.q_ts + (int64_t)(kh * 4 + hq) * a.q_hs + 8 * h;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            const f4 x0 = *reinterpret_cast<const f4*>(qr + 16 * ks);
            const f4 x1 = *reinterpret_cast<const f4*>(qr + 16 * ks + 4);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = e < 4 ? x0[e] : x1[e - 4];
                const _Float16 hi = (_Float16)x;
                qb[ks][e] = hi;
                ql[ks][e] = (_Float16)(x - (float)hi);
            }
        }
    } else {
        const uint16_t* qr = a.q16 + (int64_t)t * a.q_ts + (int64_t)(kh * 4 + hq) * a.q_hs + 8 * h;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) qb[ks] = ld_h8(qr + 16 * ks);
    }

    for (int j = j_begin; j < j_end; j++) {
        const bool more = j + 1 < j_end;
        // K of tile j has landed (V of tile j, copied after it, may still be in flight)
        asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        wave_lds_sync();
        const uint8_t* kl = st + k_lane;
        const uint8_t* vl = st + v_lane;
        const int j0 = k0 + j * PF_BK;
        f16x sv;
#pragma unroll
        for (int r = 0; r < 16; r++) sv[r] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            const h8 kop = pf_lds_h8(kl + ks * 32);
            sv = mfma32(kop, qb[ks], sv);
            if constexpr (HILO) sv = mfma32(kop, ql[ks], sv);
        }
        if (more) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // every K read of the tile is done
            wave_lds_sync();
            issue_k(j + 1);
        }
        // causal mask where a key may pass a column's position; register r holds key j0 + 8(r/4) + 4h + r%4
        if (j0 + PF_BK - 1 > off + rb) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = j0 + 8 * (r >> 2) + 4 * h + (r & 3);
                sv[r] = key <= qpos ? sv[r] : -INFINITY;
            }
        }
        float tm = sv[0];
#pragma unroll
        for (int r = 1; r < 16; r++) tm = fmaxf(tm, sv[r]);
        tm = max_xhalf(tm);
        const float tmax = tm * sc;
        float alpha = 1.0f;
        bool moved = false;
        if (tmax > m_run + 8.0f) {
            moved = m_run != -INFINITY;
            alpha = moved ? __builtin_amdgcn_exp2f(m_run - tmax) : 0.0f;
            m_run = tmax;
        }
        if (__ballot(moved)) {
            if (h == 0) bc[r32] = alpha;
            wave_lds_sync();
            f4 al[4];
#pragma unroll
            for (int gg = 0; gg < 4; gg++) al[gg] = bc_lds[w][2 * gg + h];
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float x = o[dt][r];
                    scale_acc(x, al[r >> 2][r & 3]);
                    o[dt][r] = x;
                }
        }
        l_run *= alpha;
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        h8 pa[2];
#pragma unroll
        for (int r = 0; r < 16; r++) pa[r >> 3][r & 7] = (_Float16)__builtin_amdgcn_exp2f(fmaf(sv[r], sc, -m_use));
        const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const h2 pp = {pa[k][2 * e], pa[k][2 * e + 1]};
                l_run = __builtin_amdgcn_fdot2(pp, one, l_run, false);
            }
        // V of tile j has landed (K of tile j + 1, copied after it, may still be in flight)
        if (more)
            asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        wave_lds_sync();
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const int imm0 = kk * 512 + 64 * dt;
                const h4 x0 = pf_lds_tr(vl + imm0);
                const h4 x1 = pf_lds_tr(vl + imm0 + 8 * PF_VP);
                const h8 vop = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
                o[dt] = mfma32(pa[kk], vop, o[dt]);
            }
        }
        if (more) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // every V read of the tile is done
            wave_lds_sync();
            issue_v(j + 1);
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wave_lds_sync();  // the stage's last reads are done before the merge writes O rows into it

    // Merge in wave order. Each wave leaves (m, l) per column and its O rows (column c: row c, dims at 4 d,
    // pitch VF_OP) in its own stage; then the block sums the waves' O scaled by 2^(m_w - M) and writes the
    // records of the columns that are real rows with keys in this split.
    const float l_tot = sum_xhalf(l_run);
    if (h == 0) {
        ml_lds[w][0][r32] = m_run;
        ml_lds[w][1][r32] = l_tot;
    }
    // O register r of tile dt: column 8(r/4) + 4h + r%4, dim 32 dt + r32
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int c = 8 * (r >> 2) + 4 * h + (r & 3);
            *reinterpret_cast<float*>(st + c * VF_OP + 4 * (32 * dt + r32)) = o[dt][r];
        }
    __syncthreads();
    for (int e = tid; e < 32 * 64; e += 64 * W) {
        const int c = e >> 6, d4 = e & 63, tc = rb + (c & 7), hc = c >> 3;
        if (tc >= T || k0 > off + tc) continue;
        float M = ml_lds[0][0][c];
#pragma unroll
        for (int v = 1; v < W; v++) M = fmaxf(M, ml_lds[v][0][c]);
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        float L = 0.0f;
#pragma unroll
        for (int v = 0; v < W; v++) {
            const float mv = ml_lds[v][0][c];
            const float f = mv == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mv - M);
            L = fmaf(ml_lds[v][1][c], f, L);
            const f4 x = *reinterpret_cast<const f4*>(lds + v * PF_STAGE + c * VF_OP + 16 * d4);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = fmaf(x[i], f, acc[i]);
        }
        float* rec = a.part + ((int64_t)kh * a.units + 8 * (tc + T * (s >> 3)) + (s & 7)) * DEC_PART;
        *reinterpret_cast<f4*>(rec + 8 + hc * D + 4 * d4) = acc;
        if (d4 == 0) {
            rec[hc] = M;
            rec[4 + hc] = L;
        }
    }
}

}  // namespace bn
