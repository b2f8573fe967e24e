// Causal GQA attention for T >= 2 query rows (speculative verify and prefill) on fp16 MFMA.
//
// Semantics follow attn_split.comp:9-58 + attn_combine.comp:6-21 + gate_rotate.comp:19-22 of the reference:
// row t (position off+t) of head h attends to cache rows [0, off+t+1) of kv head h/4; softmax(q.k/16) v,
// then a * sigmoid(gate). The K/V rows of the call are appended to the cache before this kernel runs.
//
// Decomposition (this kernel's own):
//   Block = 4 waves = the 4 query heads of one kv head x 32 consecutive tokens (one q-tile), so every K/V tile
//   staged in LDS serves 128 query rows. Wave w owns head 4*kh + w; lane l owns token l%32.
//   K/V tiles of 64 keys are loaded to registers one tile ahead and written to LDS (double buffer): K row-major
//   [key][256] (+16 B pad per row), V transposed [dim][64 keys] (+16 B pad) with the keys of every 16-group
//   permuted so that one ds_read_b128 gives a lane the 8 keys its PV operand needs.
//   S^T = K Q^T on v_mfma_f32_32x32x16_f16 (A = K from LDS, B = Q in registers, fp16): lane l then holds 16
//   of the 32 keys of its own query row, so the row max / sum need one cross-half shuffle.
//   Online softmax in fp32 in the log2 domain (scores scaled by log2(e)/16 after the MFMA). P (fp16) is the
//   A operand of O = P V straight from the S^T registers; O (32 rows x 256 dims, fp32) stays in registers.
//   Causal masking only on the tiles that cross the diagonal; tiles past it are not visited.
//   Longest q-tiles first, each kv head pinned to a fixed set of XCDs so its K/V stay in one XCD's L2.
//   When the q-tiles alone cannot fill the GPU, the key range of a q-tile is split; each split writes
//   (m, l, acc) per row and flash_combine_kernel merges them in split order.
#pragma once
#include "bn_device.h"

namespace bn {

constexpr int FL_BQ = 32;                      // tokens per q-tile
constexpr int FL_BK = 64;                      // keys per K/V tile
constexpr int FL_KS = 264;                     // halves per K row in LDS (256 + 8)
constexpr int FL_VS = 72;                      // halves per V^T row in LDS (64 + 8)
constexpr int FL_KBUF = FL_BK * FL_KS;         // halves per K stage (16896)
constexpr int FL_VBUF = D * FL_VS;             // halves per V stage (18432)
constexpr int FL_ROWS = 4 * FL_BQ;             // query rows per block

struct FlashArgs {
    const float* q;          // element t*q_ts + h*q_hs + d (fp32) ...
    const uint16_t* q16;     // ... or fp16 bits when non-null
    int64_t q_ts, q_hs;
    const uint16_t* kc;      // fp16 [rows][KV][256]
    const uint16_t* vc;
    const float* gate;       // element t*g_ts + h*g_hs + d, or null
    int64_t g_ts, g_hs;
    float* out;              // element t*o_ts + h*o_hs + d
    int64_t o_ts, o_hs;
    float* part_acc;         // [KV][ntq][max_splits][128 rows][256]
    float* part_ml;          // [KV][ntq][max_splits][128 rows][2]: m (log2 domain), l
    int T, off, KV, ntq;
    int ct;                  // K tiles per split
    int max_splits;
};

// position of key k (0..15) of a 16-key group inside the V^T row: keys {4h..4h+3, 8+4h..8+4h+3} -> 8h..8h+7
__device__ __forceinline__ int vperm16(int k) { return ((k & 4) << 1) | ((k & 8) >> 1) | (k & 3); }

__device__ __forceinline__ h8 lds_h8(const uint16_t* p) { return *reinterpret_cast<const h8*>(p); }

__global__ __launch_bounds__(256) void flash_kernel(FlashArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][FL_KBUF];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][FL_VBUF];
    __shared__ f4 bc_lds[4][8];  // per wave: 32 floats broadcast (alpha, then 1/l) in row order

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
    const int t0 = qt * FL_BQ;
    const int t_last = min(a.T, t0 + FL_BQ) - 1;
    const int nk = a.off + a.T;                         // cache rows that exist
    const int kt_all = (a.off + t_last + 1 + FL_BK - 1) / FL_BK;
    const int kt0 = s * a.ct;
    if (kt0 >= kt_all) return;
    const int kt1 = min(kt_all, kt0 + a.ct);
    const int64_t kvd = (int64_t)KV * D;
    const uint16_t* kb = a.kc + (int64_t)kh * D;
    const uint16_t* vb = a.vc + (int64_t)kh * D;

    // Q^T operand: lane l holds token t0 + l%32 (clamped), dims ks*16 + 8h .. +7, fp16
    const int head = kh * 4 + w;
    const int tq = t0 + r32;
    h8 qb[16];
    {
        const int tl = min(tq, a.T - 1);
        if (a.q16) {
            const uint16_t* qr = a.q16 + (int64_t)tl * a.q_ts + (int64_t)head * a.q_hs + 8 * h;
#pragma unroll
            for (int ks = 0; ks < 16; ks++) qb[ks] = ld_h8(qr + ks * 16);
        } else {
            const float* qr = a.q + (int64_t)tl * a.q_ts + (int64_t)head * a.q_hs + 8 * h;
#pragma unroll
            for (int ks = 0; ks < 16; ks++) qb[ks] = ld_f32x8_as_h8(qr + ks * 16);
        }
    }

    // tile loads (rows clamped to the existing cache rows; clamped rows are masked or never read)
    h8 kr[8], vr[2][4];
    auto load_tile = [&](int kt) {
        const int j0 = kt * FL_BK;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = tid + 256 * i, key = c >> 5, dc = c & 31;
            const int row = min(j0 + key, nk - 1);
            kr[i] = ld_h8(kb + (int64_t)row * kvd + dc * 8);
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int u = tid + 256 * i, kg = u & 15, dg = u >> 4;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = min(j0 + 4 * kg + r, nk - 1);
                vr[i][r] = ld_h8(vb + (int64_t)row * kvd + dg * 8);
            }
        }
    };
    auto store_tile = [&](int buf) {
        uint16_t* ks_ = k_lds[buf];
        uint16_t* vs_ = v_lds[buf];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = tid + 256 * i, key = c >> 5, dc = c & 31;
            *reinterpret_cast<h8*>(ks_ + key * FL_KS + dc * 8) = kr[i];
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int u = tid + 256 * i, kg = u & 15, dg = u >> 4;
            const int pb = 16 * (kg >> 2) + vperm16(4 * (kg & 3));
#pragma unroll
            for (int e = 0; e < 8; e++) {
                h4 v4 = {vr[i][0][e], vr[i][1][e], vr[i][2][e], vr[i][3][e]};
                *reinterpret_cast<h4*>(vs_ + (dg * 8 + e) * FL_VS + pb) = v4;
            }
        }
    };

    f16x o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const float sc = QK_SCALE * LOG2E;
    const int qpos = a.off + tq;  // this lane's row sees keys <= qpos

    load_tile(kt0);
    store_tile(0);
    __syncthreads();
    for (int kt = kt0; kt < kt1; kt++) {
        const int buf = (kt - kt0) & 1;
        const bool more = kt + 1 < kt1;
        if (more) load_tile(kt + 1);
        const uint16_t* ks_ = k_lds[buf];
        const uint16_t* vs_ = v_lds[buf];
        const int j0 = kt * FL_BK;

        // S^T: two 32-key halves
        f16x st[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++) {
#pragma unroll
            for (int r = 0; r < 16; r++) st[k2][r] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 16; ks++)
                st[k2] = mfma32(lds_h8(ks_ + (32 * k2 + r32) * FL_KS + ks * 16 + 8 * h), qb[ks], st[k2]);
        }
        // scale, causal mask on diagonal tiles, online softmax (log2 domain)
        const bool diag = j0 + FL_BK - 1 > a.off + t0;
        float tmax = -INFINITY;
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float x = st[k2][r] * sc;
                if (diag) {
                    const int j = j0 + 32 * k2 + 8 * (r >> 2) + 4 * h + (r & 3);
                    x = j <= qpos ? x : -INFINITY;
                }
                st[k2][r] = x;
                tmax = fmaxf(tmax, x);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = exp2f(m_run - m_use);
        float psum = 0.0f;
        h8 pa[4];
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float p = exp2f(st[k2][r] - m_use);
                psum += p;
                pa[2 * k2 + (r >> 3)][r & 7] = (_Float16)p;
            }
        l_run = l_run * alpha + psum;
        m_run = m_new;

        // rescale O rows by alpha (row of register r: 8(r/4) + 4h + r%4)
        float* bc = reinterpret_cast<float*>(bc_lds[w]);
        if (h == 0) bc[r32] = alpha;
        f4 al[4];
#pragma unroll
        for (int g = 0; g < 4; g++) al[g] = bc_lds[w][2 * g + h];
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[dt][r] *= al[r >> 2][r & 3];

        // O += P V
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                o[dt] = mfma32(pa[kk], lds_h8(vs_ + (32 * dt + r32) * FL_VS + 16 * kk + 8 * h), o[dt]);

        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

    // row totals (both lane halves hold the same row)
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    float* bc = reinterpret_cast<float*>(bc_lds[w]);
    if (h == 0) bc[r32] = a.max_splits == 1 ? l_tot : 0.0f;
    f4 lv[4];
#pragma unroll
    for (int g = 0; g < 4; g++) lv[g] = bc_lds[w][2 * g + h];

    if (a.max_splits == 1) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int t = t0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (t >= a.T) continue;
            float* op = a.out + (int64_t)t * a.o_ts + (int64_t)head * a.o_hs + r32;
            const float* zp = a.gate ? a.gate + (int64_t)t * a.g_ts + (int64_t)head * a.g_hs + r32 : nullptr;
            const float lr = lv[r >> 2][r & 3];
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                float y = o[dt][r] / lr;
                if (zp) y = gate_mul(y, zp[32 * dt]);
                op[32 * dt] = y;
            }
        }
        return;
    }
    // split partials: unnormalised rows, m and l per row
    const int64_t prow = (((int64_t)kh * ntq + qt) * a.max_splits + s) * FL_ROWS + w * FL_BQ;
    if (h == 0) {
        a.part_ml[(prow + r32) * 2] = m_run;
        a.part_ml[(prow + r32) * 2 + 1] = l_tot;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int rr = 8 * (r >> 2) + 4 * h + (r & 3);
        float* pp = a.part_acc + (prow + rr) * D + r32;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) pp[32 * dt] = o[dt][r];
    }
}

// Merge of the key splits of one (token, head) row in split order (attn_combine.comp:10-20), then the gate.
// Grid (T, H) x 64 threads; thread: dims 4*lane .. +3.
__global__ __launch_bounds__(64) void flash_combine_kernel(FlashArgs a) {
    const int t = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
    const int kh = head >> 2, w = head & 3, qt = t / FL_BQ;
    const int t_last = min(a.T, qt * FL_BQ + FL_BQ) - 1;
    const int kt_all = (a.off + t_last + 1 + FL_BK - 1) / FL_BK;
    const int ns = (kt_all + a.ct - 1) / a.ct;
    const int64_t row0 = (((int64_t)kh * a.ntq + qt) * a.max_splits) * FL_ROWS + w * FL_BQ + (t % FL_BQ);
    float M = -INFINITY;
    for (int sp = 0; sp < ns; sp++) M = fmaxf(M, a.part_ml[(row0 + (int64_t)sp * FL_ROWS) * 2]);
    float L = 0.0f;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp = 0; sp < ns; sp++) {
        const int64_t rw = row0 + (int64_t)sp * FL_ROWS;
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
