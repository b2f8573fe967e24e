// Split-KV decode attention (one query token per sequence) over an fp16 KV cache.
//
// Semantics follow attn_split.comp:9-58 + attn_combine.comp:6-21 + gate_rotate.comp:19-22 of the reference
// (query row of head h attends to cache rows [0, L) of kv head h/4, softmax(q.k / 16), gate a*sigmoid(z));
// the decomposition is this kernel's own:
//   grid (unit, kv head) x W waves. A unit serves the 4 query heads that share its kv head, so every K/V byte is
//   read once.
//   Flat order (a batch of sequences): per kv head the keys of all sequences, in order, form one stream of
//   sum_i L_i keys, cut into units of `chunk` keys, chunk ~ ceil(sum_i L_i / target) (a multiple of 16, at least
//   64 and max_len / max_splits). A unit may hold the tail of one sequence, whole sequences and the head of the
//   next (one segment each), so every unit but the last holds exactly `chunk` keys and the blocks are balanced
//   however the lengths are spread; ceil(sum_i L_i / chunk) <= target bounds the launch, and units past the last
//   exit at once. Segment (unit b, sequence i) writes partial-record slot b + i, so sequence i's records are
//   contiguous. xcd_rows (the T rows of one call): each row takes ceil(L_t / chunk) splits of its own, placed so
//   that a row's splits run on different XCDs (dec_slot). Every block derives chunk and its segments from the
//   lengths itself (a wave-wide scan over the length array, which sits in L2), so there is no planning launch and
//   a captured graph can be replayed with new device-side lengths. The split structure is a function of the
//   lengths only, so results are reproducible bit for bit.
//   QK^T: v_mfma_f32_16x16x32_f16 computes S^T = K Q^T over 16-key tiles. The A operand is the K tile read
//   straight from HBM in MFMA layout (lane: key l%16, 8 dims per k-step); the B operand holds the 4 heads'
//   query rows as an fp16 hi/lo pair (columns h and h+4, repeated in 8..15), so hi + lo carries the fp32
//   query and the scores are fp32-accurate at no extra MFMA cost.
//   Softmax: online, in the log2 domain (q pre-scaled by log2 e), fp32.
//   PV: fp32 FMAs on the VALU; each lane owns 8 dims of every other key and the 4 heads.
//   Combine: a sequence that fits one split is finished (divided and gated) by its split. Otherwise each
//   split writes (m, l, acc[256]) per head to the workspace and decode_combine_kernel, launched next on the
//   same stream, merges them (four waves per head, each over every fourth split, then the four sums in wave
//   order) and gates. The kernel boundary makes the partials visible across the XCDs' separate L2s. A merge by
//   the last block of each sequence (one launch) was built three ways and measured slower every time, for the
//   1K-key decode (8/2 heads, 17 splits) and the 8K-key one (16/4 heads, 64 splits), against 16 and 22 us with the
//   second launch: device-scope release/acquire fences per block (an L2 write-back and invalidate on gfx950) 28
//   and 190 us; records written and read with device-coherent accesses, no fences, a compare-and-swap counter 25
//   and 112 us; the same with one fetch-and-add per block 21 and 45 us. Device-scope atomics on one address
//   serialize at about 0.3 us each, more than the combine launch saves. The merge order is fixed, so results do
//   not depend on scheduling.
//   Append: when k_new/v_new are given, the new row (last key of the sequence) is taken from them, rounded
//   to fp16, used for the score and the PV product, and stored into the cache by the same split.
#pragma once
#include "bn_device.h"
#include "bn_prep.h"

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
    const uint32_t* dyn; // rows of one sequence with a device offset (graph replay): len0 is then
                         // call_off(dyn, len0 - 1) + 1, the host len0 its upper bound
    const float* gate;   // element seq*g_ss + head*g_hs + d, or null
    int64_t g_ss, g_hs;
    float* out;          // element seq*o_ss + head*o_hs + d
    int64_t o_ss, o_hs;
    const float* signs;  // [heads*256] +-1, or null; when set, out receives each row rotated: blocks of 512
                         // (heads 2j, 2j+1) times the signs, Walsh-Hadamard transformed, / sqrt(512)
    RopeParams rp;       // rp.qn set: q and k_new are raw attn_prep inputs (q_proj rows, k_proj rows) that the
                         // kernel norms and rotates in its prologue (position column: the sequence index)
    float* part;         // [KV][units][DEC_PART] (records by slot)
    int KV, nseq, max_len;
    int target;          // splits aimed at per kv head
    int max_splits;      // splits of one sequence at most
    int units;           // record slots per kv head (the stride of `part`)
    int xcd_rows;        // rows of one sequence (verify): unit 8 (t + T (s / 8)) + s % 8 is split s of row t, so the
                         // same split of every row runs on one XCD and shares its K/V rows through that L2
    int chunk;           // nonzero: keys per split, fixed by verify_kernel, which writes a record for every row and
                         // split (decode_combine_kernel then also merges rows of one split)
};

constexpr int DEC_MIN_CHUNK = 64;

// Keys per split for a batch with `sum_len` keys in total (per kv head): about sum_len / target, at least
// DEC_MIN_CHUNK, and enough that no sequence (of at most max_len keys) takes more than max_splits splits; the
// same on host and device.
__host__ __device__ inline int dec_chunk(int64_t sum_len, int target, int max_len, int max_splits) {
    int64_t c = (sum_len + target - 1) / target;
    const int64_t cs = ((int64_t)max_len + max_splits - 1) / max_splits;
    if (c < cs) c = cs;
    c = (c + 15) / 16 * 16;
    if (c < DEC_MIN_CHUNK) c = DEC_MIN_CHUNK;
    const int64_t cap = ((int64_t)max_len + 15) / 16 * 16;
    if (c > cap) c = cap;
    return (int)c;
}

// Keys per unit in flat order (a batch cut into equal runs of its concatenated keys): about sum_len / target, at
// least DEC_MIN_CHUNK and (max_len / max_splits), a multiple of 16; a unit may span several sequences, so there is
// no upper bound. Then ceil(sum_len / chunk) <= target. The same on host and device.
__host__ __device__ inline int dec_chunk_flat(int64_t sum_len, int target, int max_len, int max_splits) {
    int64_t c = (sum_len + target - 1) / target;
    const int64_t cs = ((int64_t)max_len + max_splits - 1) / max_splits;
    if (c < cs) c = cs;
    c = (c + 15) / 16 * 16;
    if (c < DEC_MIN_CHUNK) c = DEC_MIN_CHUNK;
    return (int)c;
}

// keys of sequence i; device-supplied lengths are clamped to the launch bound
__device__ __forceinline__ int dec_len(const DecodeArgs& a, int i) {
    const int len0 = a.dyn ? call_off(a.dyn, a.len0 - 1) + 1 : a.len0;
    return max(0, min(a.kv_len ? a.kv_len[i] : len0 + i * a.len_step, a.max_len));
}
__device__ __forceinline__ int64_t dec_row0(const DecodeArgs& a, int i) {
    return a.kv_off ? a.kv_off[i] : a.row0 + (int64_t)i * a.row_step;
}
__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    return x;
}
__device__ __forceinline__ int64_t wave_sum64(int64_t x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// The split structure of the batch, as seen from one wave.
// Flat order (a batch of sequences, or the rows of one call that do not use xcd_rows): the keys of all sequences, in
// order, form one stream of sum_i L_i keys per kv head, cut into units of `chunk` keys. Unit b covers stream keys
// [b chunk, (b + 1) chunk), so it may hold the tail of one sequence, whole sequences and the head of the next; each
// (unit, sequence) pair is a segment. Segment (b, i) writes record slot b + i: along the stream every step to the
// next segment raises b, i or both, so the slots are distinct, and sequence i's records are the contiguous slots
// P_i .. P_i + n_i - 1, with P_i = S_i / chunk + i (S_i its first stream key, n_i the units it touches). Every unit
// but the last holds exactly `chunk` keys, so the blocks of a launch are balanced whatever the lengths are.
// xcd_rows: the T rows of one sequence, split s of row t (chunk keys of its own) in unit and slot
// 8 (t + T (s / 8)) + s % 8.
struct DecSplit {
    int chunk, seq, P, n, L;
    int64_t S;       // stream position of the sequence's first key (flat order)
    int64_t u0, u1;  // the unit's stream keys (dec_find_unit, flat order)
    int s;           // xcd_rows: the split of `seq` that the unit works on
};

// Partial record slot of split s of sequence seq (first slot P).
__device__ __forceinline__ int dec_slot(const DecodeArgs& a, int P, int seq, int s) {
    return a.xcd_rows ? 8 * (seq + a.nseq * (s >> 3)) + (s & 7) : P + s;
}

// The batch's chunk (from its total length; the first 64 lengths are left in L0, one per lane).
__device__ __forceinline__ int dec_batch_chunk(const DecodeArgs& a, int lane, int& L0, int64_t& total) {
    if (a.nseq == 1) {  // one sequence: no wave-wide sum (its shuffles sit on every block's critical path)
        const int L = dec_len(a, 0);
        L0 = lane == 0 ? L : 0;
        total = L;
    } else {
        L0 = lane < a.nseq ? dec_len(a, lane) : 0;
        int64_t tot = L0;
        for (int base = 64; base < a.nseq; base += 64) tot += base + lane < a.nseq ? dec_len(a, base + lane) : 0;
        total = wave_sum64(tot);
    }
    if (a.chunk) return a.chunk;
    return a.xcd_rows ? dec_chunk(total, a.target, a.max_len, a.max_splits)
                      : dec_chunk_flat(total, a.target, a.max_len, a.max_splits);
}

// Flat order: the first sequence that unit b touches, with its length and stream start, and the unit's stream keys;
// xcd_rows: the row and split of unit b. seq = -1 when b is past the last unit. Sequences are scanned 64 at a time
// (one per lane).
__device__ DecSplit dec_find_unit(const DecodeArgs& a, int b, int lane) {
    DecSplit r;
    int L0;
    int64_t total;
    r.chunk = dec_batch_chunk(a, lane, L0, total);
    r.seq = -1;
    r.P = r.n = r.L = r.s = 0;
    r.S = r.u0 = r.u1 = 0;
    if (a.xcd_rows) {
        const int sb = 8 * (b / (8 * a.nseq)) + (b & 7), t = (b >> 3) % a.nseq;
        const int L = dec_len(a, t), n = (L + r.chunk - 1) / r.chunk;
        if (sb < n) {
            r.seq = t;
            r.n = n;
            r.L = L;
            r.s = sb;
        }
        return r;
    }
    r.u0 = (int64_t)b * r.chunk;
    if (r.u0 >= total) return r;
    r.u1 = min(total, r.u0 + r.chunk);
    if (a.nseq == 1) {
        r.seq = 0;
        r.L = (int)total;
        return r;
    }
    int64_t prefix = 0;
    for (int base = 0; base < a.nseq; base += 64) {
        const int Li = base == 0 ? L0 : (base + lane < a.nseq ? dec_len(a, base + lane) : 0);
        const int incl = wave_incl_scan(Li, lane);  // at most 64 lengths of 2^24: no overflow
        const int tot = __shfl(incl, 63);
        if (r.u0 < prefix + tot) {
            const uint64_t hit = __ballot(prefix + incl > r.u0);
            const int f = __builtin_ctzll(hit);
            r.seq = base + f;
            r.L = __shfl(Li, f);
            r.S = prefix + __shfl(incl, f) - r.L;
            break;
        }
        prefix += tot;
    }
    return r;
}

// The records of sequence `seq`: its first slot P and their count n (0 or 1: the split kernel finished it).
__device__ DecSplit dec_find_seq(const DecodeArgs& a, int seq, int lane) {
    DecSplit r;
    int L0;
    int64_t total;
    r.chunk = dec_batch_chunk(a, lane, L0, total);
    r.seq = seq;
    r.s = 0;
    r.S = r.u0 = r.u1 = 0;
    if (a.xcd_rows) {
        r.L = dec_len(a, seq);
        r.n = (r.L + r.chunk - 1) / r.chunk;
        r.P = 0;
        return r;
    }
    int64_t prefix = 0;
    r.L = 0;
    if (a.nseq == 1) {
        r.L = (int)total;
    } else {
        for (int base = 0; base <= seq; base += 64) {
            const int Li = base == 0 ? L0 : (base + lane < a.nseq ? dec_len(a, base + lane) : 0);
            const int incl = wave_incl_scan(Li, lane);
            if (seq < base + 64) {
                const int f = seq - base;
                r.L = __shfl(Li, f);
                r.S = prefix + __shfl(incl, f) - r.L;
                break;
            }
            prefix += __shfl(incl, 63);
        }
    }
    if (r.L > 0) {
        const int64_t b0 = r.S / r.chunk, b1 = (r.S + r.L - 1) / r.chunk;
        r.n = (int)(b1 - b0 + 1);
        r.P = (int)b0 + seq;
    } else {
        r.n = 0;
        r.P = 0;
    }
    return r;
}

__device__ __forceinline__ int64_t uniform64(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x), hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Wave-local LDS hand-off: the wave's LDS writes are complete and visible to its own lanes afterwards.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// W waves per block. A split's 16-key tiles are dealt to the waves in contiguous runs (wave w: tiles
// [w nt / W, (w+1) nt / W)); each wave keeps its own online softmax, and the block merges the W partial
// (m, l, acc) in wave order through LDS. One partial (or the finished output) per block.
// SHARED: cached K/V loads, for rows read by several units (the rows of one sequence in the XCD-aware order: the
// other rows find them in L2) and for launches of at most one block per CU (latency-bound); otherwise non-temporal
// loads stream them (a compile-time choice: a branch in the tile loop costs the streaming case 10%).
template <int W, bool SHARED = false>
__global__ __launch_bounds__(64 * W) void decode_split_kernel(DecodeArgs a) {
    __shared__ f4 p_lds[W][16];   // per wave: p[key in tile][head]
    __shared__ f4 al_lds[W];      // per wave: per-head rescale of the running accumulators
    __shared__ f4 ml_lds[W][2];   // per wave: final m, l per head
    __shared__ float acc_lds[W > 1 ? W : 1][4 * D];  // per wave: acc[head][dim] (W > 1)
    __shared__ float q_lds[4 * D];                   // attn_prep in the prologue: the group's q rows
    __shared__ float k_lds[D];                       // ... and the appended key row

    const int b = blockIdx.x, kh_ = blockIdx.y;
    const int lane_ = threadIdx.x & 63;
    const int wave = W > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
    // every argument word the block needs is requested at entry, in one round trip: left alone, the compiler
    // fetches the words that a later branch needs after that branch (a kernel-argument load takes about 0.6 us)
    asm volatile("" ::"s"(a.q), "s"(a.q16), "s"(a.kc), "s"(a.vc), "s"(a.q_ss), "s"(a.q_hs), "s"(a.gate), "s"(a.out),
                 "s"(a.part), "s"(a.k_new), "s"(a.v_new), "s"(a.signs), "s"(a.rp.qn), "s"(a.rp.kn), "s"(a.rp.pos),
                 "s"(a.rp.inv_freq), "s"(a.rp.rot));
    const DecSplit sp = dec_find_unit(a, b, lane_);
    if (sp.seq < 0) return;
    const int chunk = sp.chunk;

    // One segment: keys [sj0, sj1) of sequence seq (L keys). finished: the segment is the whole sequence, and the
    // block writes its output row; otherwise the segment's partial record goes to `slot`.
    auto segment = [&](const int seq, const int L, const int sj0, const int sj1, const bool finished, const int slot) {
        // the kv head and lane as values the compiler cannot see through: otherwise it hoists every address and
        // load that depends only on them out of the segment loop, and the kernel runs at one wave per SIMD
        int kh = kh_, lane = lane_;
        asm volatile("" : "+s"(kh), "+v"(lane));
        const int64_t row0 = dec_row0(a, seq);
        // this wave's keys [j0, j1) (empty for waves without a tile)
        const int nt = (sj1 - sj0 + 15) >> 4;
        const int j0 = sj0 + 16 * (wave * nt / W);
        const int j1 = min(sj1, sj0 + 16 * ((wave + 1) * nt / W));
        // this wave owns the appended row L-1 (none when a device offset lies past the bound: the flag is set)
        const bool has_new = a.k_new != nullptr && j1 == L && j0 < j1 && !(a.dyn && dyn_over(a.dyn, a.len0 - 1));
        const int tl = j0 + (j1 - j0 - 1) / 16 * 16;          // first key of the wave's last (maybe partial) tile
        const int64_t kvd = (int64_t)a.KV * D;
        const uint16_t* kb = a.kc + (row0 * a.KV + kh) * D;
        const uint16_t* vb = a.vc + (row0 * a.KV + kh) * D;

        const int c = lane & 15, g = lane >> 4;       // MFMA column / k-group of this lane
        const int pvr = lane >> 5, pvd = (lane & 31) * 8;  // PV layout: key parity, first dim

        float m_run = -INFINITY, l_run = 0.0f;
        float acc[4][8];
    #pragma unroll
        for (int h = 0; h < 4; h++)
    #pragma unroll
            for (int e = 0; e < 8; e++) acc[h][e] = 0.0f;

        // the first tile's K/V loads go out before the q rows are read and converted; rows past the wave's end are
        // clamped to its last row (in bounds; their scores are masked)
        auto load_k = [&](int jt, h8* kt) {
            const int r = min(jt + c, j1 - 1);
            const uint16_t* p = kb + (int64_t)r * kvd + g * 8;
    #pragma unroll
            for (int ks = 0; ks < 8; ks++) kt[ks] = SHARED ? ld_h8(p + ks * 32) : ld_h8_nt(p + ks * 32);
        };
        auto load_v = [&](int jt, h8* vt) {
    #pragma unroll
            for (int i = 0; i < 8; i++) {
                const int r = min(jt + 2 * i + pvr, j1 - 1);
                vt[i] = SHARED ? ld_h8(vb + (int64_t)r * kvd + pvd) : ld_h8_nt(vb + (int64_t)r * kvd + pvd);
            }
        };
        h8 kt[8], vt[8];
        if (j0 < j1) {
            load_k(j0, kt);
            load_v(j0, vt);
        }

        // attn_prep in the prologue (attn_prep.comp:40-56): the group's 4 q rows (wave w: heads w, w + W, ...) and,
        // in the wave that appends it, the new key row are normed and rotated into LDS
        // (the raw rows are loaded before the angles are computed, so the two overlap)
        const bool prep = a.rp.qn != nullptr;
        if (prep) {
            constexpr int NQ = (4 + W - 1) / W;
            f4 xq[NQ], xk;
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                const int h = wave + W * i;
                if (h < 4)
                    xq[i] = *reinterpret_cast<const f4*>(a.q + seq * a.q_ss + (int64_t)(kh * 4 + h) * a.q_hs + 4 * lane);
            }
            if (has_new) xk = *reinterpret_cast<const f4*>(a.k_new + seq * a.kn_ss + kh * D + 4 * lane);
            const f4 wq = *reinterpret_cast<const f4*>(a.rp.qn + 4 * lane);
            f4 cs, sn;
            rope_angles(a.rp, seq, lane, cs, sn);
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                const int h = wave + W * i;
                if (h < 4) *reinterpret_cast<f4*>(&q_lds[h * D + 4 * lane]) = norm_rope(xq[i], wq, cs, sn, a.rp.rot, lane);
            }
            if (has_new) {
                const f4 wk = *reinterpret_cast<const f4*>(a.rp.kn + 4 * lane);
                *reinterpret_cast<f4*>(&k_lds[4 * lane]) = norm_rope(xk, wk, cs, sn, a.rp.rot, lane);
            }
            __syncthreads();
        }

        if (j0 < j1) {
            // B operand: Q^T, column c = head (c&3), hi part for (c&4)==0 else lo part, k-step ks covers
            // dims ks*32 + g*8 .. +7.
            h8 qb[8];
            {
                // every q load is issued before any conversion (one wait), from whichever source the call uses
                const int64_t qo = seq * a.q_ss + (int64_t)(kh * 4 + (c & 3)) * a.q_hs + g * 8;
                const bool lo = (c & 4) != 0;
                float x[8][8];
                if (a.q16) {
                    h8 v[8];
    #pragma unroll
                    for (int ks = 0; ks < 8; ks++) v[ks] = ld_h8(a.q16 + qo + ks * 32);
    #pragma unroll
                    for (int ks = 0; ks < 8; ks++)
    #pragma unroll
                        for (int e = 0; e < 8; e++) x[ks][e] = (float)v[ks][e];
                } else {
                    f4 u[8], v[8];
                    if (prep) {
                        const float* qs = q_lds + (c & 3) * D + g * 8;
    #pragma unroll
                        for (int ks = 0; ks < 8; ks++) {
                            u[ks] = *reinterpret_cast<const f4*>(qs + ks * 32);
                            v[ks] = *reinterpret_cast<const f4*>(qs + ks * 32 + 4);
                        }
                    } else {
                        const float* qs = a.q + qo;
    #pragma unroll
                        for (int ks = 0; ks < 8; ks++) {
                            u[ks] = *reinterpret_cast<const f4*>(qs + ks * 32);
                            v[ks] = *reinterpret_cast<const f4*>(qs + ks * 32 + 4);
                        }
                    }
    #pragma unroll
                    for (int ks = 0; ks < 8; ks++)
    #pragma unroll
                        for (int e = 0; e < 4; e++) {
                            x[ks][e] = u[ks][e];
                            x[ks][e + 4] = v[ks][e];
                        }
                }
    #pragma unroll
                for (int ks = 0; ks < 8; ks++)
    #pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float y = x[ks][e] * LOG2E;
                        const _Float16 hi = (_Float16)y;
                        qb[ks][e] = lo ? (_Float16)(y - (float)hi) : hi;
                    }
            }

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
                    for (int r = 0; r < 4; r++) p_lds[wave][4 * g + r][c] = p[r];
                    if (g == 0) al_lds[wave][c] = alpha;
                }
                wave_lds_sync();
                const f4 al = al_lds[wave];
    #pragma unroll
                for (int h = 0; h < 4; h++)
    #pragma unroll
                    for (int e = 0; e < 8; e++) acc[h][e] *= al[h];
    #pragma unroll
                for (int i = 0; i < 8; i++) {
                    const f4 pv = p_lds[wave][2 * i + pvr];
    #pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float v = (float)vt[i][e];
    #pragma unroll
                        for (int h = 0; h < 4; h++) acc[h][e] = fmaf(pv[h], v, acc[h][e]);
                    }
                }
                wave_lds_sync();
            };

            // full tiles [j0, tl) with the next tile's loads in flight, then the last tile [tl, j1)
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
                // row L-1 of the last tile comes from k_new / v_new (fp16, nearest even) and is stored to the
                // cache, so a call that appends and one that finds the row cached produce the same bits. Every load
                // of the row is issued before the conversions and stores (one wait): V row slot iv of the lanes
                // whose parity matches, the K row in the lanes of MFMA row rn.
                const int rn = L - 1 - tl;  // tile row of the new key
                uint16_t* kdst = a.kc + ((row0 + L - 1) * a.KV + kh) * D;
                uint16_t* vdst = a.vc + ((row0 + L - 1) * a.KV + kh) * D;
                const int iv = (rn - pvr) >> 1;
                const bool vhit = ((rn - pvr) & 1) == 0;
                h8 vnew = vt[0];
                if (vhit) vnew = ld_f32x8_as_h8(a.v_new + seq * a.kn_ss + kh * D + pvd);
                if (c == rn) {
                    if (prep) {
    #pragma unroll
                        for (int ks = 0; ks < 8; ks++) kt[ks] = ld_f32x8_as_h8(k_lds + ks * 32 + g * 8);
                    } else {
                        const float* kn = a.k_new + seq * a.kn_ss + kh * D;
    #pragma unroll
                        for (int ks = 0; ks < 8; ks++) kt[ks] = ld_f32x8_as_h8(kn + ks * 32 + g * 8);
                    }
    #pragma unroll
                    for (int ks = 0; ks < 8; ks++) st_h8(kdst + ks * 32 + g * 8, kt[ks]);
                }
                if (vhit) {
    #pragma unroll
                    for (int i = 0; i < 8; i++)
                        if (i == iv) vt[i] = vnew;
                    st_h8(vdst + pvd, vnew);
                }
            }
            tile(kt, vt, tl, j1);
        }

        // totals over the lanes holding the same head / dims
        float l_tot = l_run + __shfl_xor(l_run, 16);
        l_tot += __shfl_xor(l_tot, 32);
    #pragma unroll
        for (int h = 0; h < 4; h++)
    #pragma unroll
            for (int e = 0; e < 8; e++) acc[h][e] += __shfl_xor(acc[h][e], 32);
        if (lane < 4) {
            ml_lds[wave][0][lane] = m_run;
            ml_lds[wave][1][lane] = l_tot;
        }

        if constexpr (W == 1) {
            wave_lds_sync();
            if (finished) {
                if (lane < 32) {
                    const f4 lsum = ml_lds[0][1];
    #pragma unroll
                    for (int h = 0; h < 4; h++) {
                        const int head = kh * 4 + h;
                        float* o = a.out + seq * a.o_ss + head * a.o_hs + pvd;
                        const float* z = a.gate ? a.gate + seq * a.g_ss + head * a.g_hs + pvd : nullptr;
                        f4 y0, y1;
    #pragma unroll
                        for (int e = 0; e < 8; e++) {
                            float y = acc[h][e] / lsum[h];
                            if (z) y = gate_mul(y, z[e]);
                            if (e < 4) y0[e] = y; else y1[e - 4] = y;
                        }
                        if (a.signs) {  // staged for the rotation below
                            const float* sg = a.signs + head * D + pvd;
                            *reinterpret_cast<f4*>(&acc_lds[0][h * D + pvd]) = y0 * *reinterpret_cast<const f4*>(sg);
                            *reinterpret_cast<f4*>(&acc_lds[0][h * D + pvd + 4]) = y1 * *reinterpret_cast<const f4*>(sg + 4);
                        } else {
                            *reinterpret_cast<f4*>(o) = y0;
                            *reinterpret_cast<f4*>(o + 4) = y1;
                        }
                    }
                }
                if (a.signs) {
                    wave_lds_sync();
                    float* o = a.out + seq * a.o_ss + (int64_t)kh * 4 * a.o_hs;
                    rotate_group_store(acc_lds[0], o, a.o_hs, 0, lane);
                    rotate_group_store(acc_lds[0], o, a.o_hs, 1, lane);
                }
                return;
            }
            float* pp = a.part + ((int64_t)kh * a.units + slot) * DEC_PART;
            if (lane < 4) {
                pp[lane] = ml_lds[0][0][lane];
                pp[4 + lane] = ml_lds[0][1][lane];
            }
            if (lane < 32) {
    #pragma unroll
                for (int h = 0; h < 4; h++) {
                    float* d = pp + 8 + h * D + pvd;
                    *reinterpret_cast<f4*>(d) = f4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
                    *reinterpret_cast<f4*>(d + 4) = f4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
                }
            }
        } else {
            // merge of the W waves in wave order: thread t handles the values v = t + 64 W k of acc[head][dim]
            if (lane < 32) {
    #pragma unroll
                for (int h = 0; h < 4; h++) {
                    float* d = &acc_lds[wave][h * D + pvd];
                    *reinterpret_cast<f4*>(d) = f4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
                    *reinterpret_cast<f4*>(d + 4) = f4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
                }
            }
            __syncthreads();
            constexpr int VPT = 4 * D / (64 * W);  // values per thread
            float* pp = finished ? nullptr : a.part + ((int64_t)kh * a.units + slot) * DEC_PART;
            // a finished row's gate logits and signs, requested together before the merge
            float zg[VPT], sg[VPT];
    #pragma unroll
            for (int k = 0; k < VPT; k++) {
                const int v = threadIdx.x + 64 * W * k, head = kh * 4 + v / D, d = v % D;
                zg[k] = finished && a.gate ? a.gate[seq * a.g_ss + head * a.g_hs + d] : 0.0f;
                sg[k] = finished && a.signs ? a.signs[head * D + d] : 0.0f;
            }
    #pragma unroll
            for (int k = 0; k < VPT; k++) {
                const int v = threadIdx.x + 64 * W * k;
                const int h = v / D, d = v % D;
                float M = -INFINITY;
    #pragma unroll
                for (int w = 0; w < W; w++) M = fmaxf(M, ml_lds[w][0][h]);
                float lsum = 0.0f, y = 0.0f;
    #pragma unroll
                for (int w = 0; w < W; w++) {
                    const float mw = ml_lds[w][0][h];
                    const float wt = mw == -INFINITY ? 0.0f : exp2f(mw - M);
                    lsum = fmaf(ml_lds[w][1][h], wt, lsum);
                    y = fmaf(acc_lds[w][v], wt, y);
                }
                if (finished) {
                    const int head = kh * 4 + h;
                    y = y / lsum;
                    if (a.gate) y = gate_mul(y, zg[k]);
                    // value v is read and staged by this thread only, so the slot in acc_lds[0] is free to reuse
                    if (a.signs)
                        acc_lds[0][v] = y * sg[k];
                    else
                        a.out[seq * a.o_ss + head * a.o_hs + d] = y;
                } else {
                    pp[8 + v] = y;
                    if (d == 0) {
                        pp[h] = M;
                        pp[4 + h] = lsum;
                    }
                }
            }
            if (finished && a.signs) {
                __syncthreads();
                if (wave < 2) rotate_group_store(acc_lds[0], a.out + seq * a.o_ss + (int64_t)kh * 4 * a.o_hs, a.o_hs, wave, lane);
            }
        }
    };

    if (a.xcd_rows) {
        const int sj0 = sp.s * chunk;
        segment(sp.seq, sp.L, sj0, min(sp.L, sj0 + chunk), sp.n == 1, b);
        return;
    }
    // flat order: the unit's segments, sequence after sequence (the loop state is wave-uniform; saying so keeps the
    // loop a uniform one, whose body the compiler allocates like straight-line code)
    int seq = __builtin_amdgcn_readfirstlane(sp.seq), L = __builtin_amdgcn_readfirstlane(sp.L);
    int64_t S = uniform64(sp.S);
    const int64_t u0 = uniform64(sp.u0), u1 = uniform64(sp.u1);
    bool any = false;
    while (true) {
        const int sj0 = (int)(max(u0, S) - S), sj1 = (int)(min(u1, S + (int64_t)L) - S);
        if (sj0 < sj1) {
            if (any) __syncthreads();  // the previous segment's LDS readers are done
            segment(seq, L, sj0, sj1, sj0 == 0 && sj1 == L, b + seq);
            any = true;
        }
        S += L;
        if (++seq >= a.nseq || S >= u1) break;
        L = __builtin_amdgcn_readfirstlane(dec_len(a, seq));
    }
}

// Merge of the split partials of one (sequence, kv head, head pair j): for each head M = max m_s,
// L = sum l_s 2^(m_s - M), out = (sum acc_s 2^(m_s - M)) / L (attn_combine.comp:10-20), then the gate and, with
// signs, the rotation of the pair's 512 elements (gate_rotate.comp:18-25). Block = 8 waves: waves 4i .. 4i+3
// merge head 2j + i, wave q of them the splits q, q + 4, q + 8, ... (lane: dims 4 lane .. +3, and one split per
// lane for the m/l terms); each wave sums its splits in order, and the four sums are added in LDS in wave order,
// so results are reproducible. Runs as its own launch after decode_split_kernel, so the partials are visible
// without device-wide fences. Grid (sequences, 2 KV).
__global__ __launch_bounds__(512) void decode_combine_kernel(DecodeArgs a) {
    __shared__ f4 o_lds[8][64];
    __shared__ float m_lds[8], l_lds[8];
    __shared__ float y_lds[2 * D];  // the pair's gated rows times the signs, when the output is rotated
    const int seq = blockIdx.x, kh = blockIdx.y >> 1, j = blockIdx.y & 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, i = wave >> 2, q = wave & 3, d0 = lane * 4;
    // the argument words in one round trip at entry (as in decode_split_kernel)
    asm volatile("" ::"s"(a.part), "s"(a.units), "s"(a.chunk), "s"(a.xcd_rows), "s"(a.gate), "s"(a.out), "s"(a.signs),
                 "s"(a.g_ss), "s"(a.g_hs), "s"(a.o_ss), "s"(a.o_hs), "s"(a.kv_len), "s"(a.dyn), "s"(a.len0),
                 "s"(a.target), "s"(a.max_splits), "s"(a.max_len), "s"(a.nseq));
    const int h = 2 * j + i, head = kh * 4 + h;
    // the gate of the wave that finishes this head goes out with the first loads (its address needs no length), so
    // its round trip overlaps the length scan's and the records' instead of following them
    f4 zg = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.gate && q == 0) zg = *reinterpret_cast<const f4*>(a.gate + seq * a.g_ss + head * a.g_hs + d0);
    const DecSplit sp = dec_find_seq(a, seq, lane);
    const int ns = sp.n;
    if (ns <= 1 && !a.chunk) return;  // written by the split kernel
    // the record of this wave's k-th split (split q + 4k)
    auto rec = [&](int k) -> const float* {
        return a.part + ((int64_t)kh * a.units + dec_slot(a, sp.P, seq, q + 4 * k)) * DEC_PART;
    };
    const int ad = 8 + h * D + d0;           // this lane's accumulators in a record
    const int nk = (ns - q + 3) >> 2;        // splits q, q + 4, ... below ns
    // the first accumulators are requested before anything waits, together with the (m, l) terms of up to 64
    // splits (one per lane), kept for the weights: a wave of up to PRE splits then needs one round trip
    constexpr int PRE = 16;
    f4 pre[PRE];
#pragma unroll
    for (int u = 0; u < PRE; u++)
        pre[u] = u < nk ? *reinterpret_cast<const f4*>(rec(u) + ad) : f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m0 = -INFINITY, l0 = 0.0f;
    if (lane < nk) {
        const float* r = rec(lane);
        m0 = r[h];
        l0 = r[4 + h];
    }
    float M = m0;
    for (int k = lane + 64; k < nk; k += 64) M = fmaxf(M, rec(k)[h]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) M = fmaxf(M, __shfl_xor(M, m));
    if (lane == 0) m_lds[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(m_lds[4 * i], m_lds[4 * i + 1]), fmaxf(m_lds[4 * i + 2], m_lds[4 * i + 3]));
    float Ls = 0.0f;
    f4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int base = 0; base < nk; base += 64) {
        const int k = base + lane;
        float w = 0.0f, lw = 0.0f;
        if (k < nk) {
            float ms = m0, ls = l0;
            if (base > 0) {
                const float* r = rec(k);
                ms = r[h];
                ls = r[4 + h];
            }
            w = ms == -INFINITY ? 0.0f : exp2f(ms - M);
            lw = ls * w;
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) lw += __shfl_xor(lw, m);
        Ls += lw;
        const int cnt = min(64, nk - base);
        int j0 = 0;
        if (base == 0) {
#pragma unroll
            for (int u = 0; u < PRE; u++)
                if (u < cnt) {
                    const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), u));
#pragma unroll
                    for (int e = 0; e < 4; e++) o[e] = fmaf(pre[u][e], wj, o[e]);
                }
            j0 = PRE;
        }
        // eight splits' loads in flight at a time, then their products in split order
        for (; j0 < cnt; j0 += 8) {
            f4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (j0 + u < cnt) v[u] = *reinterpret_cast<const f4*>(rec(base + j0 + u) + ad);
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (j0 + u < cnt) {
                    const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j0 + u));
#pragma unroll
                    for (int e = 0; e < 4; e++) o[e] = fmaf(v[u][e], wj, o[e]);
                }
        }
    }
    o_lds[wave][lane] = o;
    if (lane == 0) l_lds[wave] = Ls;
    __syncthreads();
    if (q == 0) {  // wave 4i finishes head 2j + i
        const f4 s = ((o_lds[wave][lane] + o_lds[wave + 1][lane]) + o_lds[wave + 2][lane]) + o_lds[wave + 3][lane];
        const float L = ((l_lds[wave] + l_lds[wave + 1]) + l_lds[wave + 2]) + l_lds[wave + 3];
        f4 y;
        if (a.gate) {
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = gate_mul(s[e] / L, zg[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = s[e] / L;
        }
        if (a.signs)
            *reinterpret_cast<f4*>(&y_lds[i * D + d0]) = y * *reinterpret_cast<const f4*>(a.signs + head * D + d0);
        else
            *reinterpret_cast<f4*>(a.out + seq * a.o_ss + head * a.o_hs + d0) = y;
    }
    if (a.signs) {
        __syncthreads();
        if (wave == 0) rotate_pair_store(y_lds, a.out + seq * a.o_ss + (int64_t)(kh * 4 + 2 * j) * a.o_hs, a.o_hs, lane);
    }
}

}  // namespace bn
