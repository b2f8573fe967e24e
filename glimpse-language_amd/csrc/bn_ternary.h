// Ternary packed linears: Y[T, O] (+)= X[T, K] W[O, K]^T for up to three matrices sharing X, with the LoRA up
// projection in the store (model.rs:455-639 qmm_lora / qmm / qmm_multi; kernels/qmv.glsl, qmv3.comp, qmv4.comp,
// qmvr.comp, qmvx.comp, qmm3.comp; kernels.metal:248-500, 664-709).
//
// Weight format (kernels/qmv.glsl:1-2): row n of W is K/16 uint32 words, word j holding codes of k = 16j + e at
// bits [2e, 2e+2); one fp16 scale per 128 codes, s[n * K/128 + k/128]; weight = scale * (code - 1).
//
// Two kernels:
//   tern_rows_kernel<NT> (T <= 4): VALU. Lanes take words of 8 rows at a time; per word and token the reference's
//     decode arithmetic, acc += s * (sum_e x_e * code_e - sum_e x_e) (qmv.glsl:22-35), then a wave sum.
//   tern_mfma_kernel<MT, KS> (T > 4): v_mfma_f32_32x32x16_f16 with X as A (tokens) and W as B (rows). Weights are
//     exact in fp16 ((code - 1) * scale is -s, 0, s or 2s); X is split into hi = fp16(x) rounded toward zero and
//     lo = fp16(x - hi), two MFMAs per tile, so each product carries 22 of x's 24 mantissa bits and every sum is
//     fp32: the same result class as the reference's fp32 matmuls (qmm3.comp, the Metal qmm's float MMA), not an
//     fp16 GEMM.
//     fp16's range ends at 65504: for a token whose chunk holds some |x| >= 2^15 the chunk runs a second time with
//     that token's x times 2^-16 (split hi/lo, accumulated with acc scaled by 2^-16 and back, powers of two), and
//     the first pass takes only the remainder x - 2^16 (hi' + lo'), so all of x (up to |x| ~ 4e9, small values of
//     such a token included) keeps about 22 bits; the check costs one compare per value.
//     Codes become fp16 weights through v_perm_b32 on a per-row 8-byte table of -s, 0, s, 2s (no conversion or
//     multiply per code).
//   tern_split_kernel + tern_pf_kernel (T > 32 with a workspace, bn_ternary_pf.h): the same arithmetic with x split
//     once per call.
// All write y = (add ? y + v : v) + sum_j u[j] * B[n, j] (store_post, qmv.glsl:10-15).
#pragma once
#include "bn_device.h"

namespace bn {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

struct TernMat {
    const uint32_t* w;   // [o][K/16]
    const uint16_t* s;   // [o][K/128] fp16
    float* y;            // output row t at y + t * y_ts
    const uint16_t* lb;  // LoRA B [o][lr] fp16, or null (no adapter on this member)
    int o;
    int64_t y_ts;
};

struct TernArgs {
    TernMat m[3];
    int n_mats;
    int rows;            // sum of the members' o; rows of member i follow member i - 1
    const float* x;      // token t at x + t * x_ts
    int64_t x_ts;
    int T, K;
    int add;
    const float* lu;     // LoRA u: token t, member i at lu + t * lu_ts + i * lr
    int64_t lu_ts;
    int lr;
};

// member of global row r; r becomes the member's row
__device__ __forceinline__ int tern_member(const TernArgs& a, int& r) {
    if (r < a.m[0].o) return 0;
    r -= a.m[0].o;
    if (r < a.m[1].o) return 1;
    r -= a.m[1].o;
    return 2;
}
// member i by value, through selects (a dynamic index into the kernel argument would copy it to scratch)
__device__ __forceinline__ TernMat tern_mat(const TernArgs& a, int i) {
    return i == 0 ? a.m[0] : (i == 1 ? a.m[1] : a.m[2]);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// y = (add ? y + v : v) + LoRA (qmv.glsl:10-15 store_post, lora_acc summed in j order)
__device__ __forceinline__ void tern_store(const TernArgs& a, const TernMat& m, int mi, int t, int n, float v) {
    float* y = m.y + (int64_t)t * m.y_ts + n;
    float yv = a.add ? *y + v : v;
    if (a.lr > 0 && m.lb) {
        const float* u = a.lu + (int64_t)t * a.lu_ts + (int64_t)mi * a.lr;
        const uint16_t* b = m.lb + (int64_t)n * a.lr;
        float acc = 0.0f;
        for (int j = 0; j < a.lr; ++j) acc = fmaf(u[j], h2f(b[j]), acc);
        yv = yv + acc;
    }
    *y = yv;
}

__device__ __forceinline__ float wave_sum_f32(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

constexpr int TERN_ROWS_WAVE = 4;  // rows per wave of tern_rows_kernel (block: 4 waves, 16 rows)

// Sums of 4 values over the wave: lane l ends with the total of value (l >> 4) & 3 (7 exchanges instead of 24:
// each step hands the partner the half of the values it does not keep).
__device__ __forceinline__ float wave_sum4(const float (&v)[4], int lane) {
    const bool up = lane & 32;
    const float a = __shfl_xor(up ? v[0] : v[2], 32), b = __shfl_xor(up ? v[1] : v[3], 32);
    const float k0 = (up ? v[2] : v[0]) + a, k1 = (up ? v[3] : v[1]) + b;
    const bool b4 = lane & 16;
    float x = (b4 ? k1 : k0) + __shfl_xor(b4 ? k0 : k1, 16);
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// T = NT <= 4 tokens. Each wave: 4 rows of one member; lane l takes words j = l, l + 64, ..., the next word's
// codes, scales and x loaded while the current one is summed.
// KH waves share a row group and split its words (wave h of the group takes words 64 h + lane + 64 KH i); their sums
// meet in LDS in wave order. Block: 4 waves = 4 / KH row groups of 4 rows.
template <int NT, int KH = 1>
__global__ __launch_bounds__(256) void tern_rows_kernel(TernArgs a) {
    constexpr int R = TERN_ROWS_WAVE;
    __shared__ float red[KH > 1 ? 4 : 1][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kh = wave % KH;
    const int r0g = (blockIdx.x * (4 / KH) + wave / KH) * R;
    const bool live = r0g < a.rows;
    if (KH == 1 && !live) return;  // no barriers below when KH == 1
    int r0 = live ? r0g : 0;
    const int mi = tern_member(a, r0);
    const TernMat m = tern_mat(a, mi);
    const int K = a.K, kw = K >> 4, kg = K >> 7;
    const uint32_t* wp = m.w + (int64_t)r0 * kw;
    const uint16_t* sp = m.s + (int64_t)r0 * kg;
    float acc[R][NT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[r][t] = 0.0f;
    uint32_t wn[R];
    uint16_t sn[R];
    f4 xn[NT][4];
    auto load = [&](int j) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wn[r] = wp[(int64_t)r * kw + j];
            sn[r] = sp[(int64_t)r * kg + (j >> 3)];
        }
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) xn[t][q] = reinterpret_cast<const f4*>(a.x + (int64_t)t * a.x_ts + 16 * j)[q];
    };
    const int jl = 64 * kh + lane;
    if (jl < kw) load(jl);
    for (int j = jl; j < kw; j += 64 * KH) {
        uint32_t wc[R];
        float sc[R], xv[NT][16], xs[NT];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wc[r] = wn[r];
            sc[r] = h2f(sn[r]);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xv[t][4 * q + e] = xn[t][q][e];
                    s += xn[t][q][e];
                }
            xs[t] = s;
        }
        if (j + 64 * KH < kw) load(j + 64 * KH);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // code e = 4b + s sits in byte b of (wd >> 2s) & 0x03030303 (one v_cvt_f32_ubyte per code)
            float c[16];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const uint32_t q = (wc[r] >> (2 * s)) & 0x03030303u;
#pragma unroll
                for (int b = 0; b < 4; ++b) c[4 * b + s] = (float)((q >> (8 * b)) & 0xFFu);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; ++e) d = fmaf(xv[t][e], c[e], d);
                acc[r][t] = fmaf(sc[r], d - xs[t], acc[r][t]);
            }
        }
    }
    // lanes 16 r (+ t) hold row r's sums; lanes 16 r + t store token t
    float mine = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float v[4] = {acc[0][t], acc[1][t], acc[2][t], acc[3][t]};
        const float sum = wave_sum4(v, lane);
        if ((lane & 15) == t) mine = sum;
    }
    if constexpr (KH > 1) {
        red[wave][lane] = mine;
        __syncthreads();
        if (!live || kh != 0) return;
#pragma unroll
        for (int h = 1; h < KH; ++h) mine += red[wave + h][lane];
    }
    if ((lane & 15) < NT) tern_store(a, m, mi, lane & 15, r0 + (lane >> 4), mine);
}

// ---- MFMA kernel --------------------------------------------------------------------------------------------
constexpr int TERN_KC = 64;  // k per staged chunk (4 MFMA k-steps of 16)
// prefill kernel shape: 32-token tiles per wave and waves per SIMD it is compiled for
#ifndef BN_TERN_PF_MT
#define BN_TERN_PF_MT 2
#endif
#ifndef BN_TERN_PF_OCC
#define BN_TERN_PF_OCC 3
#endif
#ifndef BN_TERN_PF_RG
#define BN_TERN_PF_RG 4
#endif
#ifndef BN_TERN_PF_KC
#define BN_TERN_PF_KC 64
#endif

// The four weights (code - 1) * s of one row and scale group as a v_perm_b32 table: lo holds the low bytes of the
// fp16 entries for codes 0..3 (-s, 0, s, 2s), hi their high bytes. 2s = s + s is exact wherever (code - 1) * s is
// finite in fp16.
struct TernTab {
    uint32_t lo, hi;
};
__device__ __forceinline__ TernTab tern_table(uint16_t sbits) {
    const _Float16 s = __builtin_bit_cast(_Float16, sbits);
    const uint32_t p = (uint32_t)sbits | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(s + s)) << 16);
    const uint32_t ng = (uint32_t)sbits ^ 0x8000u;  // -s
    // byte sources: 4, 5 = -s; 0, 1 = s; 2, 3 = 2s; 0x0c = zero
    return {__builtin_amdgcn_perm(ng, p, 0x02000c04u), __builtin_amdgcn_perm(ng, p, 0x03010c05u)};
}

// 8 codes of a word as fp16 weights: slots 2i, 2i+1 = codes 4kg + i, 8 + 4kg + i (the A layout below), which sit at
// bits 2i of bytes kg and 2 + kg. dup = kg ? 0x03030101 : 0x02020000 repeats those bytes as [b, b, b', b'];
// (d >> 2i) & 0x03030303 | 0x04000400 is then the selector [c, c + 4, c', c' + 4]: lo[c], hi[c], lo[c'], hi[c'],
// the two fp16 weights of the slot pair.
__device__ __forceinline__ h8 tern_decode8(uint32_t w, uint32_t dup, TernTab t) {
    const uint32_t d = __builtin_amdgcn_perm(0u, w, dup);
    h8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // one v_and_or_b32 (its VOP3 form takes no literal: the mask comes in an SGPR, the OR term in a VGPR)
        uint32_t sel;
        asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(sel) : "v"(d >> (2 * i)), "s"(0x03030303u), "v"(0x04000400u));
        const h2 v = __builtin_bit_cast(h2, __builtin_amdgcn_perm(t.hi, t.lo, sel));
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}

// A block whose waves each stage their own K range (KS > 1, one row group) orders its LDS writes and reads within
// the wave (LDS instructions of one wave complete in order); a block whose waves share the staged tile syncs.
template <int KS>
__device__ __forceinline__ void tern_sync() {
    if constexpr (KS > 1) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
        __syncthreads();
    }
}

// LDS row of token row m in block k = 2q + kg of a staged chunk: m XOR a per-block mask, a bijection inside each
// 16-row group. Staging writes 8 (or 16) consecutive lanes to the same m in consecutive blocks, which start BM * 16
// bytes apart (the same banks); the mask spreads them over distinct 16-byte bank slots, and the A-operand reads
// (32 consecutive m per block) stay a permutation of slots within every 8- and 16-lane group.
template <int NQ>
__device__ __forceinline__ int tern_swz(int m, int k) {
    if constexpr (NQ == 4) return m ^ (k | ((m & 1) << 3));
    else return m ^ (k & 15);
}

#ifndef BN_TERN_XCD_GROUP
#define BN_TERN_XCD_GROUP 4
#endif

// Block -> (row tile rt, token tile tt). Workgroups are dealt to the 8 XCDs round robin (block b on XCD b % 8), and
// each XCD has its own L2. When the token tiles divide evenly, XCD x takes the token tiles x, x + 8, ... in groups of
// G (BN_TERN_XCD_GROUP by default; tern_pf_kernel's 128-token blocks take half as many, so a group spans the same
// tokens) and runs every row tile of a group before the next group, the group's token tiles of one row tile on
// consecutive blocks: each x tile is fetched into one L2 (and stays there while the row tiles pass), and each row
// tile's codes serve the group from that L2. Otherwise row tiles run fastest (token tile by token tile).
template <int BM, int G = BN_TERN_XCD_GROUP>
__device__ __forceinline__ void tern_tile(int b, int row_tiles, int T, int& rt, int& tt) {
    const int ntt = (T + BM - 1) / BM;
    if (G < 1 || (ntt & 7) || ntt < 16) {
        rt = b % row_tiles;
        tt = b / row_tiles;
        return;
    }
    const int x = b & 7, k = b >> 3, nx = ntt >> 3;   // nx token tiles per XCD
    const int group = k / (G * row_tiles), rem = k - group * G * row_tiles;
    const int gg = min(G, nx - group * G);             // token tiles in this group (the last may be short)
    rt = rem / gg;
    tt = x + 8 * (group * G + rem % gg);
}

// ---- x as fp16 hi/lo pairs ----------------------------------------------------------------------------------
constexpr float TERN_BIG = 32768.0f;  // a token with a value this large in a chunk takes the scaled pass

// whether the token of a unit (8 of its values; its 2 nq units on 2 nq consecutive lanes) has a value >= TERN_BIG
template <int NQ>
__device__ __forceinline__ bool tern_token_big(f4 va, f4 vb, bool valid) {
    bool b = false;
#pragma unroll
    for (int s = 0; s < 4; ++s) b |= fabsf(va[s]) >= TERN_BIG || fabsf(vb[s]) >= TERN_BIG;
    int t = valid && b;
#pragma unroll
    for (int o = 1; o < 2 * NQ; o <<= 1) t |= __shfl_xor(t, o);
    return t != 0;
}
// hi = x rounded toward zero to fp16 (for |x| < 2^16 at or above fp16's normal range: x with its low 13 mantissa bits
// dropped; below it hi keeps fewer bits and lo the rest), lo = fp16(x - hi) with x - hi exact in fp32: hi + lo
// carries 22 of x's 24 significant bits
__device__ __forceinline__ void tern_split2(float x0, float x1, _Float16& h0, _Float16& h1, _Float16& l0,
                                            _Float16& l1) {
    const h2 h = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x0, x1));
    h0 = h[0];
    h1 = h[1];
    l0 = (_Float16)(x0 - (float)h[0]);
    l1 = (_Float16)(x1 - (float)h[1]);
}
// The part of x a token with a value >= TERN_BIG keeps for the main pass: x - 2^16 (hi' + lo'), with (hi', lo') the
// split of x 2^-16 that the scaled pass multiplies (exact: the two are within a factor of two, or the scaled part is
// zero). Together the passes carry every value to about 22 bits, small ones included.
__device__ __forceinline__ float tern_remainder(float x) {
    _Float16 h, h_, l, l_;
    tern_split2(x * (1.0f / 65536.0f), 0.0f, h, h_, l, l_);
    return x - ((float)h + (float)l) * 65536.0f;
}
// The 8 values of a unit (va = k + 0..3, vb = k + 8..11) as hi and lo slots (slot 2s = va[s], 2s + 1 = vb[s]).
// mode 0: x; 1: the remainder of a large token; 2: x 2^-16 (the scaled pass); 3: zeros
__device__ __forceinline__ void tern_split8(f4 va, f4 vb, int mode, h8& hi, h8& lo) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        float xa = va[s], xb = vb[s];
        if (mode == 1) {
            xa = tern_remainder(xa);
            xb = tern_remainder(xb);
        } else if (mode == 2) {
            xa *= 1.0f / 65536.0f;
            xb *= 1.0f / 65536.0f;
        } else if (mode == 3) {
            xa = xb = 0.0f;
        }
        _Float16 h0, h1, l0, l1;
        tern_split2(xa, xb, h0, h1, l0, l1);
        hi[2 * s] = h0;
        hi[2 * s + 1] = h1;
        lo[2 * s] = l0;
        lo[2 * s + 1] = l1;
    }
}
// max |x| over 8 values (v_max3 with |.| operands: a NaN gives no >= TERN_BIG and stays on the mode-0 path, which
// carries it through)
__device__ __forceinline__ void tern_absmax8(float& mx, f4 va, f4 vb) {
#pragma unroll
    for (int s = 0; s < 4; ++s) asm("v_max3_f32 %0, |%1|, |%2|, %0" : "+v"(mx) : "v"(va[s]), "v"(vb[s]));
}

// MT 32-token tiles x 2 32-row tiles per wave; KS waves split K (their partial sums meet in LDS in ks order), RG
// waves split rows (KS > 1 only with RG = 1). Block: 64 * KS * RG threads, 32 * MT tokens x 64 * RG rows.
//
// A layout in LDS, per k-split group: hi[KC / 16 q][2 kg][32 MT m][8 slots] fp16, then lo the same. Slot i of (q, kg, m)
// holds x[m][k0 + 16q + 4kg + 8(i & 1) + (i >> 1)], the k order tern_decode8 gives the B operand, so each lane's A
// operand (m = lane % 32, kg = lane / 32) is one 16-byte LDS read.
template <int MT, int KS, int RG, int OCC = 1, int KC = TERN_KC>
__global__ __launch_bounds__(64 * KS * RG, OCC) void tern_mfma_kernel(TernArgs a, int row_tiles) {
    constexpr int NQ = KC / 16;        // MFMA k-steps per chunk
    static_assert(KC == 64 || KC == 128, "a chunk lies inside one 128-column scale group");
    static_assert(KS * RG <= 8 && (KS == 1 || (RG == 1 && MT == 1)), "split-K blocks are one token tile, one row group");
    constexpr int BM = 32 * MT;        // tokens per block
    constexpr int GROUP_H = 2 * NQ * 2 * BM * 8;  // fp16 per k-split group (hi and lo): NQ q * 2 kg * BM * 8 * 2
    // one buffer, two syncs per chunk: a second buffer costs registers and occupancy (3 -> 2 waves per SIMD for
    // the prefill shape) and measured slower on MI355X
    __shared__ __attribute__((aligned(16))) _Float16 lds[KS * GROUP_H];
    // per wave (KS = 1): whether it staged a token with a value >= TERN_BIG in the current chunk. Written before and read
    // after the chunk's staging barrier; the next chunk writes only after the barrier that opens it, which every
    // wave reaches after its reads.
    __shared__ __attribute__((aligned(16))) int big_flag[KS == 1 ? RG : 1];
    static_assert(KS * GROUP_H * 2 <= 65536, "LDS");
    static_assert(KS * 32 * MT * 64 * 4 <= KS * GROUP_H * 2 || KS == 1, "reduction buffer fits the A buffer");

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rg = wave / KS, ks = wave % KS;
    int rt, tt;
    tern_tile<BM>((int)blockIdx.x, row_tiles, a.T, rt, tt);
    const int t0 = tt * BM;
    const int rbase_g = (rt * RG + rg) * 64;  // first global row of this wave
    const bool active = rbase_g < a.rows;
    int rbase = active ? rbase_g : 0;
    const int mi = tern_member(a, rbase);
    const TernMat m = tern_mat(a, mi);

    const int K = a.K, kw = K >> 4, kg = K >> 7;
    const int klen = K / KS, kbase = ks * klen, nchunk = klen / KC;

    // staging: group thread gt of 64 * RG takes units u = gt + i * 64 * RG, u = (m * NQ + q) * 2 + kgu; the 2 NQ
    // units of one token in a chunk sit on 2 NQ consecutive lanes of the same i
    constexpr int GT = 64 * RG, UPT = 2 * NQ * BM / GT;
    static_assert(GT % (2 * NQ) == 0, "a token's units stay inside one wave");
    const int gt = rg * 64 + lane;
    _Float16* glds = lds + ks * GROUP_H;
    f4 xa[UPT], xb[UPT];
    auto load_x = [&](int c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const int u = gt + i * GT;
            const int mm = u / (2 * NQ), q = (u >> 1) % NQ, kgu = u & 1;
            // token rows past T are not staged: their A rows only feed outputs that are not stored. Prefill blocks
            // (KS = 1) load them anyway from row T - 1 (in bounds), so that the next chunk's loads are unconditional
            // and stay in flight (a conditional load leaves register copies that the compiler waits for right after
            // issuing the next loads); split-K blocks of a few tokens skip them.
            if (KS == 1 || t0 + mm < a.T) {
                const float* p = a.x + (int64_t)min(t0 + mm, a.T - 1) * a.x_ts + kbase + c * KC + 16 * q + 4 * kgu;
                xa[i] = *reinterpret_cast<const f4*>(p);
                xb[i] = *reinterpret_cast<const f4*>(p + 8);
            }
        }
    };
    auto stage_unit = [&](int mm, int q, int kgu, f4 va, f4 vb, int mode) __attribute__((always_inline)) {
        h8 hi, lo;
        tern_split8(va, vb, mode, hi, lo);
        const int off = ((q * 2 + kgu) * BM + tern_swz<NQ>(mm, q * 2 + kgu)) * 8;
        *reinterpret_cast<h8*>(glds + off) = hi;
        *reinterpret_cast<h8*>(glds + 2 * NQ * BM * 8 + off) = lo;
    };
    // stages the loaded chunk (tokens with a value >= TERN_BIG: their remainders); returns whether this lane staged
    // such a token
    auto store_x = [&]() __attribute__((always_inline)) {
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < UPT; ++i) tern_absmax8(mx, xa[i], xb[i]);
        // the common case, no such value in any unit of the wave (a unit past T, which KS = 1 loads from row T - 1,
        // can only send the wave to the general path below)
        if (__ballot(mx >= TERN_BIG) == 0) {
#pragma unroll
            for (int i = 0; i < UPT; ++i) {
                const int u = gt + i * GT;
                const int mm = u / (2 * NQ), q = (u >> 1) % NQ, kgu = u & 1;
                if (t0 + mm < a.T) stage_unit(mm, q, kgu, xa[i], xb[i], 0);
            }
            return false;
        }
        bool any_big = false;
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const int u = gt + i * GT;
            const int mm = u / (2 * NQ), q = (u >> 1) % NQ, kgu = u & 1;
            const bool valid = t0 + mm < a.T;
            const bool big = tern_token_big<NQ>(xa[i], xb[i], valid);
            any_big |= big;
            if (valid) stage_unit(mm, q, kgu, xa[i], xb[i], big ? 1 : 0);
        }
        return any_big;
    };
    // the scaled pass of chunk c: x reloaded, tokens with a value >= TERN_BIG staged times 2^-16, the others as zeros
    auto store_big = [&](int c) __attribute__((always_inline)) {
#pragma unroll 1
        for (int i = 0; i < UPT; ++i) {
            const int u = gt + i * GT;
            const int mm = u / (2 * NQ), q = (u >> 1) % NQ, kgu = u & 1;
            const bool valid = t0 + mm < a.T;
            const float* p = a.x + (int64_t)min(t0 + mm, a.T - 1) * a.x_ts + kbase + c * KC + 16 * q + 4 * kgu;
            const f4 va = *reinterpret_cast<const f4*>(p), vb = *reinterpret_cast<const f4*>(p + 8);
            const bool big = tern_token_big<NQ>(va, vb, valid);
            if (valid) stage_unit(mm, q, kgu, va, vb, big ? 2 : 3);
        }
    };

    // B: lane (n = lane % 32, kgl = lane / 32) of row tile nt reads row rbase + 32 nt + n
    const int n = lane & 31, kgl = lane >> 5;
    const uint32_t* wrow[2];
    const uint16_t* srow[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int64_t row = rbase + 32 * nt + n;
        wrow[nt] = m.w + row * kw + kbase / 16;
        srow[nt] = m.s + row * kg;
    }
    u4 wv[2][NQ / 4];
    uint16_t sv_next[2] = {0, 0};  // the next chunk's scales, loaded with its codes
    auto load_w = [&](int c) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
            for (int h = 0; h < NQ / 4; ++h) wv[nt][h] = *reinterpret_cast<const u4*>(wrow[nt] + c * (KC / 16) + 4 * h);
            sv_next[nt] = srow[nt][(kbase + c * KC) >> 7];
        }
    };

    f16x acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][nt][e] = 0.0f;

    const uint32_t dup = kgl ? 0x03030101u : 0x02020000u;
    // inactive waves (rows past the last matrix) load member 0's first rows, in bounds, and do not use them
    load_x(0);
    load_w(0);
    for (int c = 0; c < nchunk; ++c) {
        tern_sync<KS>();  // the previous chunk's A reads are done
        const bool staged_big = store_x();
        u4 wcur[2][NQ / 4];
#pragma unroll
        for (int h = 0; h < NQ / 4; ++h) {
            wcur[0][h] = wv[0][h];
            wcur[1][h] = wv[1][h];
            // the copy happens here, before the next chunk's loads are issued (its wait then covers only the loads
            // of this chunk, which had the previous chunk's compute to land)
            asm volatile("" ::"v"(wcur[0][h][0]), "v"(wcur[0][h][1]), "v"(wcur[0][h][2]), "v"(wcur[0][h][3]),
                         "v"(wcur[1][h][0]), "v"(wcur[1][h][1]), "v"(wcur[1][h][2]), "v"(wcur[1][h][3]));
        }
        TernTab tab[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) tab[nt] = tern_table(sv_next[nt]);
        asm volatile("" ::"v"(tab[0].lo), "v"(tab[0].hi), "v"(tab[1].lo), "v"(tab[1].hi));
        // the staging is complete (block-wide for KS = 1, where the waves share it; wave-wide otherwise), and
        // whether any token of it was held back for the scaled pass
        bool chunk_big;
        if constexpr (KS > 1) {
            tern_sync<KS>();
            chunk_big = __ballot(staged_big) != 0;
        } else {
            const bool wave_big = __ballot(staged_big) != 0;
            if (lane == 0) big_flag[rg] = wave_big;
            __syncthreads();
            int f = 0;
#pragma unroll
            for (int r = 0; r < RG; ++r) f |= big_flag[r];
            chunk_big = f != 0;
        }
        if (KS == 1 || c + 1 < nchunk) {
            const int cn = min(c + 1, nchunk - 1);  // prefill blocks: the last chunk reloads itself (unused)
            load_x(cn);
            load_w(cn);
        }
        // the chunk's MFMAs over the staged hi/lo tiles
        auto mfma_chunk = [&](const u4 (&wc)[2][NQ / 4], const TernTab (&tb)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                h8 b[2];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) b[nt] = tern_decode8(wc[nt][q >> 2][q & 3], dup, tb[nt]);
                h8 ah[MT], al[MT];
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const int off = ((q * 2 + kgl) * BM + tern_swz<NQ>(32 * i + n, q * 2 + kgl)) * 8;
                    ah[i] = *reinterpret_cast<const h8*>(glds + off);
                    al[i] = *reinterpret_cast<const h8*>(glds + 2 * NQ * BM * 8 + off);
                }
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) acc[i][nt] = mfma32(ah[i], b[nt], acc[i][nt]);
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) acc[i][nt] = mfma32(al[i], b[nt], acc[i][nt]);
            }
        };
        if (active) mfma_chunk(wcur, tab);
        if (chunk_big) {
            // rare: some token had a value beyond fp16's range in this chunk (decided uniformly for the threads that
            // share the staging). Its x, times 2^-16, is multiplied into acc times 2^-16, and acc is scaled back:
            // acc + 2^16 (x 2^-16) W^T, with every scaling a power of two (exact).
            tern_sync<KS>();
            store_big(c);
            tern_sync<KS>();
            if (active) {
                // the chunk's codes and scales again (the staged copies are not kept alive for this rare pass)
                u4 wr[2][NQ / 4];
                TernTab tr[2];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
                    for (int h = 0; h < NQ / 4; ++h) wr[nt][h] = *reinterpret_cast<const u4*>(wrow[nt] + c * (KC / 16) + 4 * h);
                    tr[nt] = tern_table(srow[nt][(kbase + c * KC) >> 7]);
                }
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) acc[i][nt] *= 1.0f / 65536.0f;
                mfma_chunk(wr, tr);
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) acc[i][nt] *= 65536.0f;
            }
        }
    }

    // C layout: acc[i][nt][j] = (token 32 i + 8 (j / 4) + 4 (lane / 32) + j % 4, row 32 nt + lane % 32)
    if constexpr (KS == 1) {
        if (!active) return;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int t = t0 + 32 * i + 8 * (j >> 2) + 4 * kgl + (j & 3);
                if (t < a.T)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) tern_store(a, m, mi, t, rbase + 32 * nt + n, acc[i][nt][j]);
            }
    } else {
        // partial tiles of the KS waves (one row group, MT = 1): red[ks][32 tokens][64 rows]
        float* red = reinterpret_cast<float*>(lds);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int tl = 8 * (j >> 2) + 4 * kgl + (j & 3);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) red[(ks * 32 + tl) * 64 + 32 * nt + n] = acc[0][nt][j];
        }
        __syncthreads();
        if (!active) return;
        // thread p sums outputs p, p + 256, ... of the 32 x 64 tile in ks order
        for (int p = threadIdx.x; p < 32 * 64; p += 64 * KS) {
            const int tl = p >> 6, col = p & 63;
            if (t0 + tl >= a.T) continue;
            float v = red[p];
#pragma unroll
            for (int k2 = 1; k2 < KS; ++k2) v += red[k2 * 32 * 64 + p];
            tern_store(a, m, mi, t0 + tl, rbase + col, v);
        }
    }
}

}  // namespace bn
