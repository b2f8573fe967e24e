// Ternary prefill GEMM with x split once per call: bn_ternary_matmul with T > 32 and a workspace (model.rs:455-596
// qmm_lora / qmm_multi over a prompt; kernels/qmm3.comp).
//
// tern_split_kernel: one block per (64-token tile, 64-column chunk) writes the chunk's x as the 16 KB that the GEMM's
// MFMAs read: the hi slots, then the lo slots, each [q 4][kg 2][m' 64][8 fp16] with m' = tern_swz<4>(m, 2q + kg),
// slot i of (q, kg, m) = x[t0 + m][64 c + 16 q + 4 kg + 8 (i & 1) + (i >> 1)] (the k order tern_decode8 gives the
// weights), split by tern_split8. Tokens past T are zeros. A token with some |x| >= 2^15 in the chunk keeps its
// remainder there and the tile's flag word is set: the GEMM then runs that chunk's scaled pass from x itself, as
// tern_mfma_kernel does.
//
// tern_pf_kernel<S, OCC, MT>: S = 2 copy stages, OCC blocks per CU, MT 32-token tiles per wave. Block = 4 waves x 64
// rows (256 rows) x 32 MT tokens (MT / 2 x tiles); for each 64-column chunk every wave copies a quarter of each x tile,
// its 64 rows' code words and their scale words into one of the 2 LDS stages with global_load_lds, one chunk ahead,
// spread among the current chunk's 16 MT MFMAs (MT token tiles x 2 row tiles x 4 k-steps x hi/lo) instead of issued
// as a burst before them (2-3% faster on the 4B q/k/v and o_proj prefills). The copies hold no VGPRs and the block
// splits nothing: what is left on the VALU is the weight decode, once per code word and block, so MT = 4 halves it
// per MFMA (2 stages of 37 KB: two blocks per CU; MT = 2 with 2 stages of 21 KB: three). One barrier per chunk: past
// it, the copies of every wave for the chunk have landed (each wave waited for its own first) and every wave is done
// with the previous chunk's stage, which the copies issued next then fill.
//
// The sums are those of tern_mfma_kernel for the same shapes (same split, same k order, same MFMA order): the two
// give identical results.
#pragma once
#include "bn_ternary.h"

namespace bn {

constexpr int TPF_BM = 64;                                    // tokens per tile
constexpr int TPF_KC = 64;                                    // columns per chunk
constexpr int TPF_NQ = TPF_KC / 16;                           // MFMA k-steps per chunk
constexpr int TPF_TILE = 2 * TPF_NQ * 2 * TPF_BM * 16;        // bytes of one (token tile, chunk): hi, then lo

// (token tile, chunk) tiles of a call; the workspace holds them, then one flag word per tile
__host__ __device__ inline size_t tern_pf_tiles(int T, int K) {
    return (size_t)((T + TPF_BM - 1) / TPF_BM) * (size_t)(K / TPF_KC);
}
inline size_t tern_pf_work_bytes(int T, int K) { return tern_pf_tiles(T, K) * (TPF_TILE + 4); }

__global__ __launch_bounds__(256) void tern_split_kernel(const float* __restrict__ x, int64_t x_ts, int T, int K,
                                                         uint8_t* __restrict__ work) {
    const int nchunk = K / TPF_KC;
    const int tile = (int)blockIdx.x, tt = tile / nchunk, c = tile - tt * nchunk, t0 = tt * TPF_BM;
    _Float16* out = reinterpret_cast<_Float16*>(work + (size_t)tile * TPF_TILE);
    uint32_t* flag = reinterpret_cast<uint32_t*>(work + (size_t)gridDim.x * TPF_TILE) + tile;
    // 512 units (m, q, kg), two per thread: the 8 units of a token sit on 8 consecutive lanes
    f4 va[2], vb[2];
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int u = (int)threadIdx.x + 256 * i, mm = u >> 3, q = (u >> 1) & 3, kgu = u & 1;
        const float* p = x + (int64_t)min(t0 + mm, T - 1) * x_ts + c * TPF_KC + 16 * q + 4 * kgu;
        va[i] = *reinterpret_cast<const f4*>(p);
        vb[i] = *reinterpret_cast<const f4*>(p + 8);
        if (t0 + mm >= T) va[i] = vb[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        tern_absmax8(mx, va[i], vb[i]);
    }
    const bool wave_big = __ballot(mx >= TERN_BIG) != 0;  // uniform: the token checks below run only when needed
    bool any_big = false;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int u = (int)threadIdx.x + 256 * i, mm = u >> 3, q = (u >> 1) & 3, kgu = u & 1;
        bool big = false;
        if (wave_big) big = tern_token_big<TPF_NQ>(va[i], vb[i], true);
        any_big |= big;
        h8 hi, lo;
        tern_split8(va[i], vb[i], big ? 1 : 0, hi, lo);
        const int off = ((q * 2 + kgu) * TPF_BM + tern_swz<TPF_NQ>(mm, q * 2 + kgu)) * 8;
        *reinterpret_cast<h8*>(out + off) = hi;
        *reinterpret_cast<h8*>(out + TPF_TILE / 4 + off) = lo;
    }
    const int f = __syncthreads_or(any_big);
    if (threadIdx.x == 0) *flag = f != 0;
}

typedef __attribute__((address_space(3))) void tpf_lds_t;

// 16 (4) bytes per lane from global memory into LDS at lds + 16 lane (4 lane). The two copy stages are separate
// arrays, so the compiler can tell one stage's copies from the other stage's operand reads and schedules them
// together; the kernel orders a stage's copies before its reads itself (s_waitcnt vmcnt, then the block barrier).
__device__ __forceinline__ void tpf_copy16(const void* g, const uint8_t* lds) {
    __builtin_amdgcn_global_load_lds(g, (tpf_lds_t*)const_cast<uint8_t*>(lds), 16, 0, 0);
}
__device__ __forceinline__ void tpf_copy4(const void* g, const uint8_t* lds) {
    __builtin_amdgcn_global_load_lds(g, (tpf_lds_t*)const_cast<uint8_t*>(lds), 4, 0, 0);
}

// copies per wave and chunk: 4 per 64-token x tile, 1 of code words, 1 of scale words
__host__ __device__ constexpr int tpf_copies(int MT) { return 4 * (MT / 2) + 2; }
// stage bytes: the block's x tiles (MT / 2 of them), the code words (4 waves x 64 rows x 16 B), the scale words
__host__ __device__ constexpr int tpf_stage(int MT) { return (MT / 2) * TPF_TILE + 4 * 1024 + 4 * 256; }

template <int S, int C>
__device__ __forceinline__ void tpf_wait_barrier() {
    static_assert(S == 2 || S == 3, "stages");
    // this wave's copies of the current chunk have landed (the S - 2 later chunks' copies may be in flight), then
    // every wave's
    if constexpr (S == 2)
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(C) : "memory");
}

// MT 32-token tiles per wave: MT = 2 covers one 64-token x tile per block, MT = 4 two (each code word decoded once
// feeds twice the MFMAs)
template <int S, int OCC, int MT = 2>
__global__ __launch_bounds__(256, OCC) void tern_pf_kernel(TernArgs a, int row_tiles, const uint8_t* __restrict__ work) {
    static_assert(MT == 2 || MT == 4, "token tiles per wave");
    static_assert(S == 2, "two copy stages");
    constexpr int BM = 32 * MT, NQ = TPF_NQ, KC = TPF_KC, NX = MT / 2;
    constexpr int STAGE = tpf_stage(MT), ST_W = NX * TPF_TILE, ST_S = ST_W + 4 * 1024;
    // the two stages are separate arrays, so that the compiler can tell a stage's copies from the other's reads
    __shared__ __attribute__((aligned(16))) uint8_t lds0[STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t lds1[STAGE];
    const int lane = (int)threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    int rt, tt;
    tern_tile<BM, (BN_TERN_XCD_GROUP * 64 / BM > 0 ? BN_TERN_XCD_GROUP * 64 / BM : 1)>((int)blockIdx.x, row_tiles,
                                                                                       a.T, rt, tt);
    const int t0 = tt * BM;
    const int rbase_g = (rt * 4 + wave) * 64;  // first global row of this wave
    const bool active = rbase_g < a.rows;
    int rbase = active ? rbase_g : 0;          // inactive waves copy member 0's first rows (in bounds, unused)
    const int mi = tern_member(a, rbase);
    const TernMat m = tern_mat(a, mi);
    const int K = a.K, kw = K >> 4, kg = K >> 7, nchunk = K / KC;
    const int nxt = (a.T + TPF_BM - 1) / TPF_BM;  // 64-token x tiles of the call
    // x tile u of the block: 64-token tile NX tt + u (a tile past the last repeats the last: its tokens are not
    // stored)
    const uint8_t* tiles[NX];
    const uint32_t* flags[NX];
#pragma unroll
    for (int u = 0; u < NX; ++u) {
        const int xt = min(NX * tt + u, nxt - 1);
        tiles[u] = work + (size_t)xt * nchunk * TPF_TILE;
        flags[u] = reinterpret_cast<const uint32_t*>(work + tern_pf_tiles(a.T, K) * TPF_TILE) + (size_t)xt * nchunk;
    }

    // the copies of chunk j into stage st
    const uint8_t* wsrc = reinterpret_cast<const uint8_t*>(m.w + (int64_t)(rbase + lane) * kw);  // row rbase + lane
    const uint16_t* ssrc = m.s + (int64_t)(rbase + lane) * kg;
    auto issue = [&](int j, const uint8_t* sb) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NX; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                tpf_copy16(tiles[u] + (size_t)j * TPF_TILE + wave * 4096 + i * 1024 + lane * 16,
                           sb + u * TPF_TILE + wave * 4096 + i * 1024);
        tpf_copy16(wsrc + j * 16, sb + ST_W + wave * 1024);  // the row's 4 code words of the chunk
        // the 4-byte word holding the row's scale of the chunk (the scale array is 4-byte aligned with an even count)
        const uintptr_t sp = reinterpret_cast<uintptr_t>(ssrc + ((j * KC) >> 7));
        tpf_copy4(reinterpret_cast<const void*>(sp & ~(uintptr_t)3), sb + ST_S + wave * 256);
    };
    auto chunk_big = [&](int j) __attribute__((always_inline)) {
        uint32_t f = 0;
#pragma unroll
        for (int u = 0; u < NX; ++u) f |= flags[u][j];
        return f != 0;
    };

    // whether some chunk of this token tile holds a value >= TERN_BIG (its scaled pass), read before the copies
    int big_local = 0;
    for (int j = lane; j < nchunk; j += 64) big_local |= chunk_big(j);
    const bool tile_big = __ballot(big_local) != 0;
    issue(0, lds0);

    const int n = lane & 31, kgl = lane >> 5;
    const uint32_t dup = kgl ? 0x03030101u : 0x02020000u;
    f16x acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][nt][e] = 0.0f;

    // the chunk's MFMAs over the stage's hi/lo tiles
    auto mfma_chunk = [&](const uint8_t* sb, const u4 (&wc)[2], const TernTab (&tb)[2]) __attribute__((always_inline)) {
        const _Float16* xl = reinterpret_cast<const _Float16*>(sb);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            h8 b[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) b[nt] = tern_decode8(wc[nt][q], dup, tb[nt]);
            h8 ah[MT], al[MT];
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int off = (i >> 1) * (TPF_TILE / 2) +
                                ((q * 2 + kgl) * TPF_BM + tern_swz<NQ>(32 * (i & 1) + n, q * 2 + kgl)) * 8;
                ah[i] = *reinterpret_cast<const h8*>(xl + off);
                al[i] = *reinterpret_cast<const h8*>(xl + TPF_TILE / 4 + off);
            }
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) acc[i][nt] = mfma32(ah[i], b[nt], acc[i][nt]);
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) acc[i][nt] = mfma32(al[i], b[nt], acc[i][nt]);
            // the next chunk's copies (issued before the chunk in program order) go out one after every MT of
            // the k-step's 4 MT MFMAs, 3 per k-step: a burst of them after the barrier held back the first MFMAs
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, MT, 0);                 // MT MFMAs
                if (g < 3) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one copy
            }
        }
    };

    // chunk c from stage sb while chunk c + 1 is copied into nb, the stage chunk c - 1 used
    auto step = [&](int c, uint8_t* sb, uint8_t* nb) __attribute__((always_inline)) {
        tpf_wait_barrier<S, tpf_copies(MT)>();
        // code words of rows n and 32 + n, and their scales
        u4 wc[2];
        TernTab tab[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int r = 32 * nt + n;
            wc[nt] = *reinterpret_cast<const u4*>(sb + ST_W + wave * 1024 + r * 16);
            const int half = (int)(((int64_t)(rbase + r) * kg + ((c * KC) >> 7)) & 1);
            tab[nt] = tern_table(*reinterpret_cast<const uint16_t*>(sb + ST_S + wave * 256 + r * 4 + half * 2));
        }
        // every wave runs the MFMAs (an inactive wave's sums are not stored), so that the copies and the MFMAs
        // are one piece of straight-line code for the scheduler
        issue(min(c + 1, nchunk - 1), nb);
        mfma_chunk(sb, wc, tab);
        if (tile_big && chunk_big(c)) {
            // rare: some token of the tile has a value beyond fp16's range in this chunk (uniform over the block).
            // Its x, times 2^-16, is multiplied into acc times 2^-16, and acc is scaled back: acc + 2^16 (x 2^-16) W^T,
            // every scaling a power of two (exact). The stage's x tiles are free once every wave is past its MFMAs;
            // the copies that refill the stage wait for the next chunk's barrier.
            __syncthreads();
            _Float16* xl = reinterpret_cast<_Float16*>(sb);
#pragma unroll 1
            for (int i = 0; i < MT; ++i) {
                const int u = (int)threadIdx.x + 256 * i, mm = u >> 3, q = (u >> 1) & 3, kgu = u & 1;
                const bool valid = t0 + mm < a.T;
                const float* p = a.x + (int64_t)min(t0 + mm, a.T - 1) * a.x_ts + c * KC + 16 * q + 4 * kgu;
                const f4 va = *reinterpret_cast<const f4*>(p), vb = *reinterpret_cast<const f4*>(p + 8);
                const bool big = tern_token_big<NQ>(va, vb, valid);
                h8 hi, lo;
                tern_split8(va, vb, big ? 2 : 3, hi, lo);
                const int off = (mm >> 6) * (TPF_TILE / 2) +
                                ((q * 2 + kgu) * TPF_BM + tern_swz<NQ>(mm & 63, q * 2 + kgu)) * 8;
                *reinterpret_cast<h8*>(xl + off) = hi;
                *reinterpret_cast<h8*>(xl + TPF_TILE / 4 + off) = lo;
            }
            __syncthreads();
            if (active) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) acc[i][nt] *= 1.0f / 65536.0f;
                mfma_chunk(sb, wc, tab);
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) acc[i][nt] *= 65536.0f;
            }
        }
    };
    for (int c = 0; c < nchunk; c += 2) {
        step(c, lds0, lds1);
        if (c + 1 < nchunk) step(c + 1, lds1, lds0);
    }
    // the last copies (repeats of the last chunk into free stages) land before the block's LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // C layout: acc[i][nt][j] = (token 32 i + 8 (j / 4) + 4 (lane / 32) + j % 4, row 32 nt + lane % 32)
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
}

}  // namespace bn
