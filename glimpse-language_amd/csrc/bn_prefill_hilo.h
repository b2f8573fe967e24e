// Causal GQA prefill for long prompts whose query rows come as fp32: the scores keep (nearly) q's full precision.
//
// Semantics follow attn_split.comp:9-58 + attn_combine.comp:6-21 + gate_rotate.comp:19-25 of the reference, as
// prefill_kernel (same arguments, same results within fp32 rounding): row t (position off+t) of head h attends to
// cache rows [0, off+t+1) of kv head h/4; softmax(q.k/16) v, then a * sigmoid(gate), optionally rotated.
//
// prefill_kernel multiplies fp16 q. An fp32 q rounded to fp16 moves a score by about 2^-12 |q||k|, which at scores
// of tens (peaky heads) shows in the output. Here q is split as hi = fp16(q), lo = fp16(q - hi) and S^T = K hi^T +
// K lo^T (two MFMAs per k-step), so the scores keep about 22 of q's 24 bits. The low part takes 64 more registers
// per lane than prefill_kernel's two waves per SIMD can hold, so this kernel runs one wave per SIMD and hides the
// latencies by software pipelining instead of by a second wave:
//   - K/V tiles of 32 keys go HBM/L2 -> LDS by global_load_lds through a ring of 4 stages, three tiles ahead, in
//     prefill_kernel's padded row-pair layout (the same operand addressing);
//   - per tile the wave computes S^T(j + 1) on the MFMA units while the VALU turns S^T(j) into P(j), then O += P(j)
//     V(j); the LDS operand reads are issued a few MFMAs ahead of their use (scheduling groups);
//   - O stays in the accumulation registers for the whole loop.
// Measured on MI355X (4096 rows, 16/4 heads): 248-282 us, against 171-178 us for prefill_kernel on the same rows
// given as fp16 (the hi/lo product adds half again the MFMA work). Run on fp16 q, this design measured 194-226 us,
// slower than prefill_kernel: one wave per SIMD issues LDS reads at about half the rate of two (130 against 260
// bytes per cycle per CU for ds_read_b128), so fp16 q stays on prefill_kernel.
#pragma once
#include "bn_prefill.h"

namespace bn {

constexpr int PH_STAGES = 4;           // K/V stages in LDS: the tile in use, the next one, two in flight
constexpr int PH_OP = 1040;             // row pitch (bytes) of a wave's output rows in LDS at the epilogue
#ifndef PH_KAHEAD
#define PH_KAHEAD 6                     // K operand reads in flight ahead of their MFMA
#endif
#ifndef PH_VAHEAD
#define PH_VAHEAD 4                     // V operand read pairs in flight ahead of their MFMA
#endif


// One block per q-tile: 4 waves, one per SIMD, wave w = query head 4 kh + w over the q-tile's 32 tokens. Each wave
// has the SIMD's whole register file (amdgpu_waves_per_eu 1): O (128), Q^T hi and lo (64 each), two S^T tiles and
// the operand reads in flight. The K/V tiles go through a ring of 4 stages (tile j in stage
// j % 4, copied three tiles ahead); one barrier per tile says that tile j + 1 has landed and that every wave has
// left tile j - 1, whose stage the copy of tile j + 3 then reuses. Tile j + 3's 8 copies go out one after every
// second k-step of S^T(j + 1) (a burst of them after the barrier left the SIMD without MFMAs for their issue time:
// 4-5% slower). Per tile the wave computes S^T(j + 1) = K(j + 1)
// Q^T on the MFMA units while the VALU turns S^T(j) into P(j) (one k-step of each at a time), then O += P(j) V(j),
// the operand reads a few MFMAs ahead of their use.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void prefill_hilo_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[PH_STAGES * PF_STAGE];
    __shared__ f4 bc_lds[4][16];  // per wave: 64 floats broadcast in row order

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, r32 = lane & 31;
    const int KV = a.KV, ntq = a.ntq;

    // block -> (kv head, q-tile): longest q-tiles (highest index) first, each kv head on a fixed set of XCDs
    int kh, qt;
    {
        const int b = blockIdx.x, nb = KV * ntq;
        int idx;
        if (8 % KV == 0 && nb % 8 == 0) {
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
    const int nk = off + a.T;                         // cache rows that exist
    const int nt = (off + t_last + PF_BK) / PF_BK;    // key tiles the q-tile attends to
    const int64_t kvd = (int64_t)KV * D;
    const uint16_t* kb = a.kc + (int64_t)kh * D;
    const uint16_t* vb = a.vc + (int64_t)kh * D;
    const int head = kh * 4 + w;

    // Q^T hi and lo straight from memory, before the copies (which count on the same vmcnt): lane l holds token
    // t0 + l % 32 (clamped), dims 16 ks + 8 h .. +7
    h8 qb[16], ql[16];
    {
        const int tq = min(t0 + r32, a.T - 1);
        const float* qr = a.q + (int64_t)tq * a.q_ts + (int64_t)head * a.q_hs + 8 * h;
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
    }
    // The loads have landed; the empty asm statements then redefine Q^T, so the compiler's own waits for these loads
    // (which would count the tile copies issued next) end here.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int ks = 0; ks < 16; ks++) {
        asm volatile("" : "+v"(qb[ks]));
        asm volatile("" : "+v"(ql[ks]));
    }

    // Tile copies: wave w moves row pairs 4w .. 4w+3 of K and of V (8 copies per tile); copy c of tile jt: K (c even)
    // or V (c odd) of row pair 4 w + c / 2, lane l loading row 32 jt + p + 16 (l / 32), clamped to the cache's last row
    // (those keys are masked), 16-byte chunk l % 32, into LDS pair p at byte 16 l.
    auto tile_copy = [&](int jt, uint8_t* st, int c) __attribute__((always_inline)) {
        const int j0 = jt * PF_BK, lim = nk - 1 - j0, p = 4 * w + (c >> 1);
        const uint32_t go = (uint32_t)(min(p + 16 * h, lim) * (int)kvd + r32 * 8) * 2u;
        if (c & 1)
            pf_copy16(reinterpret_cast<const char*>(vb + (int64_t)j0 * kvd) + go, st + PF_KB + p * PF_VP);
        else
            pf_copy16(reinterpret_cast<const char*>(kb + (int64_t)j0 * kvd) + go, st + p * PF_KP);
    };
    // tiles 0, 1, 2 into stages 0, 1, 2 (a tile past the last repeats the last: its stage is never read as such), so
    // that every tile step finds the same copies in flight
#pragma unroll
    for (int j = 0; j < PH_STAGES - 1; j++)
#pragma unroll
        for (int c = 0; c < 8; c++) tile_copy(min(j, nt - 1), lds + j * PF_STAGE, c);

    f16x o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float sc = QK_SCALE * LOG2E;
    const int qpos = off + t0 + r32;  // this lane's row sees keys <= qpos
    const int k_lane = (r32 & 15) * PF_KP + (r32 >> 4) * 512 + h * 16;
    const int vs = lane & 15, vnh = (lane >> 4) & 1;
    const int v_lane = PF_KB + (4 * h + (vs >> 2)) * PF_VP + 32 * vnh + 8 * (vs & 3);
    float* bc = reinterpret_cast<float*>(bc_lds[w]);

    // tile 0 landed (tiles 1 and 2 may still be in flight), for every wave; then S^T(0)
    asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
    f16x s_cur;
    {
        const uint8_t* kl = lds + k_lane;
#pragma unroll
        for (int r = 0; r < 16; r++) s_cur[r] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            const h8 kop = pf_lds_h8(kl + ks * 32);
            s_cur = mfma32(kop, qb[ks], s_cur);
            s_cur = mfma32(kop, ql[ks], s_cur);
        }
    }

    // Tile j: S^T(j + 1) from stage j + 1 (computed also after the last tile, from a stage whose copies are done,
    // and dropped), P(j) from S^T(j), O += P(j) V(j) from stage j.
    for (int j = 0; j < nt; j++) {
        // tile j + 1 landed (tile j + 2's copies may be in flight), and every wave is done with tile j - 1, whose
        // stage takes tile j + 3 (a repeat of the last tile past the end), copied during the S^T(j + 1) MFMAs below
        asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
        const int jc = min(j + 3, nt - 1);
        uint8_t* cst = lds + ((j + 3) & (PH_STAGES - 1)) * PF_STAGE;
        const uint8_t* cur = lds + (j & (PH_STAGES - 1)) * PF_STAGE;
        const uint8_t* nxt = lds + ((j + 1) & (PH_STAGES - 1)) * PF_STAGE;

        // K(j + 1) operand reads run KA k-steps ahead of their MFMAs; the first ones hide behind the row max
        constexpr int KA = PH_KAHEAD, VA = PH_VAHEAD;
        const uint8_t* kl = nxt + k_lane;
        h8 kop[16];
#pragma unroll
        for (int ks = 0; ks < KA; ks++) kop[ks] = pf_lds_h8(kl + ks * 32);

        // the row max of S(j); causal mask on tiles that cross the diagonal (register r: key j0 + 8 (r/4) + 4 h + r%4)
        const int j0 = j * PF_BK;
        if (j0 + PF_BK - 1 > off + t0) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = j0 + 8 * (r >> 2) + 4 * h + (r & 3);
                s_cur[r] = key <= qpos ? s_cur[r] : -INFINITY;
            }
        }
        float tm = s_cur[0];
#pragma unroll
        for (int r = 1; r < 16; r++) tm = fmaxf(tm, s_cur[r]);
        tm = max_xhalf(tm);
        const float tmax = tm * sc;  // log2 domain
        // Conditional rescale: m_run moves only when the row's tile max exceeds it by more than 8 (log2 units);
        // otherwise p = 2^(x - m_run) <= 256 stays well inside fp16 and the final division by l cancels the common
        // factor. Rows with no key yet (m_run = -inf) have O = 0 and just take the max.
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

        // S(j + 1) on the MFMA units while the VALU turns S(j) into P(j), one k-step at a time; the first V(j)
        // operand reads start in the last k-steps
        f16x s_next;
#pragma unroll
        for (int r = 0; r < 16; r++) s_next[r] = 0.0f;
        h8 pa[2];
        h4 vx[16][2];
        const uint8_t* vl = cur + v_lane;
        auto v_read = [&](int i) {  // PV step i: keys 16 (i / 8) .. +15, dims 32 (i % 8) .. +31
            const int imm0 = (i >> 3) * 512 + 64 * (i & 7);
            vx[i][0] = pf_lds_tr(vl + imm0);
            vx[i][1] = pf_lds_tr(vl + imm0 + 8 * PF_VP);
        };
        // The scheduling groups fix the order per k-step (its LDS reads, its two MFMAs, four VALU instructions), so
        // the reads stay KA (V: VA) steps ahead; left alone, the compiler moves each read next to its MFMA.
#pragma unroll
        for (int ks = 0; ks < 16; ks++) {
            if (ks + KA < 16) kop[ks + KA] = pf_lds_h8(kl + (ks + KA) * 32);
            if (ks + VA >= 16) v_read(ks + VA - 16);
            s_next = mfma32(kop[ks], qb[ks], s_next);
            s_next = mfma32(kop[ks], ql[ks], s_next);
            pa[ks >> 3][ks & 7] = (_Float16)__builtin_amdgcn_exp2f(fmaf(s_cur[ks], sc, -m_use));
            if (ks + KA < 16 && ks + VA >= 16) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
            else if (ks + KA < 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            else if (ks + VA >= 16) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x402, 4, 0);
            if (ks & 1) {  // one copy after every second k-step's MFMAs, which stay ahead of it
                tile_copy(jc, cst, ks >> 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const h2 pp = {pa[k][2 * e], pa[k][2 * e + 1]};
                l_run = __builtin_amdgcn_fdot2(pp, one, l_run, false);
            }
        // O += P(j) V(j) over the 32 keys: two 16-key steps; V operand rows 16 kk + 8 rd + 4 h + (l % 16) / 4
#pragma unroll
        for (int i = 0; i < 16; i++) {
            if (i + VA < 16) v_read(i + VA);
            const h8 vop = __builtin_shufflevector(vx[i][0], vx[i][1], 0, 1, 2, 3, 4, 5, 6, 7);
            o[i & 7] = mfma32(pa[i >> 3], vop, o[i & 7]);
            if (i == 0) __builtin_amdgcn_sched_group_barrier(0x402, 8, 0);
            if (i + VA < 16) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        s_cur = s_next;
    }

    // Epilogue. O / l goes to LDS as each wave's [32 tokens][256 dims] (pitch PH_OP), then rows are read back 16
    // bytes per lane for coalesced gated stores, or, with signs, per (token, head pair) for the rotation.
    const float l_tot = sum_xhalf(l_run);
    if (h == 0) bc[r32] = 1.0f / l_tot;
    f4 lv[4];
#pragma unroll
    for (int gg = 0; gg < 4; gg++) lv[gg] = bc_lds[w][2 * gg + h];
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last tile steps' copies (repeats) have landed
    __syncthreads();  // every wave is done with the stages
    uint8_t* orow = lds + w * 32 * PH_OP;
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int tl = 8 * (r >> 2) + 4 * h + (r & 3);
            *reinterpret_cast<float*>(orow + tl * PH_OP + 4 * (32 * dt + r32)) = o[dt][r] * lv[r >> 2][r & 3];
        }
    __syncthreads();
    if (!a.signs) {
#pragma unroll 4
        for (int tl = 0; tl < PF_BQ; tl++) {
            const int t = t0 + tl;
            if (t >= a.T) break;
            f4 y = *reinterpret_cast<const f4*>(orow + tl * PH_OP + 16 * lane);
            if (a.gate) {
                const f4 z = *reinterpret_cast<const f4*>(a.gate + (int64_t)t * a.g_ts + (int64_t)head * a.g_hs + 4 * lane);
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = gate_mul_fast(y[e], z[e]);
            }
            __builtin_nontemporal_store(y, reinterpret_cast<f4*>(a.out + (int64_t)t * a.o_ts + (int64_t)head * a.o_hs +
                                                               4 * lane));  // streamed out, as in prefill_kernel
        }
        return;
    }
    // rotation: (token tl, head pair p) blocks, 16 per wave; lane l holds dims 4l .. 4l+3 of heads 2p and 2p + 1
#pragma unroll 1
    for (int k = w; k < 2 * PF_BQ; k += 4) {
        const int tl = k >> 1, p = k & 1, t = t0 + tl;
        if (t >= a.T) break;
        float v[8];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int hw = 2 * p + i, hd = kh * 4 + hw;
            f4 y = *reinterpret_cast<const f4*>(lds + hw * 32 * PH_OP + tl * PH_OP + 16 * lane);
            if (a.gate) {
                const f4 z = *reinterpret_cast<const f4*>(a.gate + (int64_t)t * a.g_ts + (int64_t)hd * a.g_hs + 4 * lane);
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = gate_mul_fast(y[e], z[e]);
            }
            y *= *reinterpret_cast<const f4*>(a.signs + (int64_t)hd * D + 4 * lane);
#pragma unroll
            for (int c = 0; c < 4; c++) v[4 * i + c] = y[c];
        }
        fwht512_wave(v, lane);
        float* o_ = a.out + (int64_t)t * a.o_ts + (int64_t)(kh * 4 + 2 * p) * a.o_hs;
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_nontemporal_store(f4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]} * INV_SQRT512,
                                        reinterpret_cast<f4*>(o_ + i * a.o_hs + 4 * lane));
    }
}

}  // namespace bn
