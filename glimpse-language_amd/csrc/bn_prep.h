// The steps either side of the attention product: attn_prep (q/k RMS-norm, interleaved mRoPE, fp16 K/V append)
// before it and gate_rotate (sigmoid gate, sign flip, 512-point Walsh-Hadamard transform) after it.
//
// Semantics follow kernels/attn_prep.comp:29-59 and kernels/gate_rotate.comp:11-26 with fwht512 of
// kernels/common.glsl:55-72 in the reference; the decompositions are this file's own (one wave per head row,
// reductions and butterflies across the wave with lane shuffles, no LDS).
#pragma once
#include "bn_device.h"
#include "bn_lora.h"

namespace bn {

// The parameters of attn_prep's norm and rotation, shared by prep_kernel and the attention kernels that apply
// it in their prologue (qn == null: the caller's q and k rows are already normed and rotated).
struct RopeParams {
    const float* qn;         // [256] q norm weight
    const float* kn;         // [256] k norm weight
    const int32_t* pos;      // [3][npos] mRoPE positions (t, h, w rows); row t of a call is position column t
    const float* inv_freq;   // [rot / 2]
    int npos, rot, s1, s2;
};

// Position column t's rotation of lane l's dims 4l .. 4l+3 (d < rot; pairs d, d + rot/2, pair index
// i = d mod rot/2): position row sel = 1 if i % 3 == 1 and i < 3 s1, 2 if i % 3 == 2 and i < 3 s2, else 0
// (attn_prep.comp:51); angle pos[sel][t] * inv_freq[i] in fp32. The same for every q and k head of the token.
// One sincosf per pair index, not four per lane: lane j computes pairs j and j + 64 (those below rot/2), then
// every lane fetches its four dims' values from the lane holding their pair index. Lanes with d >= rot get
// cos 1, sin 0. Called by all 64 lanes of the wave (the shuffles read every lane).
__device__ __forceinline__ void rope_angles(const RopeParams& rp, int t, int lane, f4& cs, f4& sn) {
    const int half = rp.rot >> 1, d0 = 4 * lane;
    float c[2] = {1.0f, 1.0f}, s[2] = {0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int i = lane + 64 * j;
        if (i < half) {
            const int sel = (i % 3 == 1 && i < 3 * rp.s1) ? 1 : ((i % 3 == 2 && i < 3 * rp.s2) ? 2 : 0);
            const float ang = (float)rp.pos[sel * rp.npos + t] * rp.inv_freq[i];
            sincosf(ang, &s[j], &c[j]);
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int i = half ? (d0 + e) % half : 0;
        float ce = __shfl(c[0], i & 63), se = __shfl(s[0], i & 63);
        if (half > 64) {  // uniform across the wave
            const float c1 = __shfl(c[1], i & 63), s1 = __shfl(s[1], i & 63);
            ce = i < 64 ? ce : c1;
            se = i < 64 ? se : s1;
        }
        cs[e] = d0 < rp.rot ? ce : 1.0f;
        sn[e] = d0 < rp.rot ? se : 0.0f;
    }
}

// One head row held by a wave (lane l: dims 4l .. 4l+3): x * (1 / sqrt(sum x^2 / 256 + 1e-6)) * w (a wave-wide
// sum), then on dims d < rot: x' = x cos - x[d + rot/2] sin (first half), x cos + x[d - rot/2] sin (second half),
// with the partner element from lane l +- rot/8 (rot is a multiple of 8, so a lane's four dims sit on one side
// of rot/2). All 64 lanes take part.
__device__ __forceinline__ f4 norm_rope(f4 x, f4 w, f4 cs, f4 sn, int rot, int lane) {
    const int d0 = 4 * lane;
    float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
    const float r = 1.0f / sqrtf(ss / 256.0f + 1e-6f);
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = x[e] * r * w[e];
    const int half = rot >> 1;
    if (d0 < rot) {
        // the partner lanes are all inside this branch
        const int pl = d0 < half ? lane + (half >> 2) : lane - (half >> 2);
        f4 xp;
#pragma unroll
        for (int e = 0; e < 4; e++) xp[e] = __shfl(x[e], pl);
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = d0 < half ? x[e] * cs[e] - xp[e] * sn[e] : x[e] * cs[e] + xp[e] * sn[e];
    }
    return x;
}

struct PrepArgs {
    const float* qp;         // q rows: element t*qp_ts + h*qp_hs + d (the q half of the q_proj output)
    int64_t qp_ts, qp_hs;
    const float* kp;         // [T][KV][256]
    const float* vp;         // [T][KV][256]
    RopeParams rp;           // npos = T
    float* q;                // element t*q_ts + h*q_hs + d: fp32 ...
    uint16_t* q16;           // ... or fp16 bits when non-null; both null: the q rows are skipped
    int64_t q_ts, q_hs;
    uint16_t* kc;            // fp16 [cap][KV][256]: rows off .. off+T-1 written
    uint16_t* vc;
    const uint32_t* dyn;     // device offset (graph replay) or null; off is then its upper bound
    int T, off, H, KV;
};

// One head row of token t: q heads [0, H), k heads [H, H+KV), v heads [H+KV, H+2KV); lane l holds dims
// 4l .. 4l+3 (x, already loaded; w the norm weights of those dims, cs/sn the token's rotation). q and k: norm
// and rotation (norm_rope); v: copied. k and v are rounded to fp16 (nearest even) into cache row off + t.
__device__ __forceinline__ void prep_row(const PrepArgs& a, int off, int t, int hh, f4 x, f4 w, f4 cs, f4 sn,
                                         int lane, bool store_kv) {
    const int H = a.H, KV = a.KV, d0 = 4 * lane;
    if (hh >= H + KV) {
        const h4 y = {(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
        if (store_kv) *reinterpret_cast<h4*>(a.vc + ((int64_t)(off + t) * KV + (hh - H - KV)) * D + d0) = y;
        return;
    }
    x = norm_rope(x, w, cs, sn, a.rp.rot, lane);
    if (hh < H) {  // q rows stream out non-temporally (4-6% faster for long prompts than ordinary stores)
        if (a.q16) {
            const h4 y = {(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
            __builtin_nontemporal_store(y, reinterpret_cast<h4*>(a.q16 + t * a.q_ts + hh * a.q_hs + d0));
        } else {
            __builtin_nontemporal_store(x, reinterpret_cast<f4*>(a.q + t * a.q_ts + hh * a.q_hs + d0));
        }
    } else if (store_kv) {
        const h4 y = {(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
        *reinterpret_cast<h4*>(a.kc + ((int64_t)(off + t) * KV + (hh - H)) * D + d0) = y;
    }
}

// Grid (T, G) x PW waves: block (t, y) = token t; wave w takes head rows h_first + R y + w, + PW, ... (PB of
// them, R = PW PB), then the same R rows further on by R G (G > 1 splits a few tokens' rows over more CUs), with
// all PB loads issued before the first is used (one row per wave left too few bytes in flight per CU to reach
// the HBM rate). The first rows' loads go out before the norm weights and the token's sin/cos are fetched and
// computed, so that work overlaps their latency. h_first = H when no q output is asked for (K/V rows only).
// Long prompts take 4 waves x 4 rows (fewer registers than 6 rows per wave, so 6 blocks per CU); a few tokens
// take 8 waves x 3 rows, all 24 rows of a 16/4-head token in flight in one block.
template <int PW, int PB>
__global__ __launch_bounds__(64 * PW) void prep_kernel(PrepArgs a) {
    const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.H, KV = a.KV, nh = H + 2 * KV, d0 = 4 * lane;
    const int h_first = (a.q || a.q16) ? 0 : H;
    const int off = call_off(a.dyn, a.off);
    const bool store_kv = !dyn_over(a.dyn, a.off);  // past the bound no K/V row is written (the flag is set)
    const int64_t kvd = (int64_t)KV * D;
    constexpr int R = PW * PB;
    auto load = [&](int h0, f4* x) {
#pragma unroll
        for (int b = 0; b < PB; b++) {
            const int hh = h0 + PW * b;
            if (hh < H)
                x[b] = *reinterpret_cast<const f4*>(a.qp + t * a.qp_ts + hh * a.qp_hs + d0);
            else if (hh < H + KV)
                x[b] = *reinterpret_cast<const f4*>(a.kp + t * kvd + (hh - H) * D + d0);
            else if (hh < nh)
                x[b] = *reinterpret_cast<const f4*>(a.vp + t * kvd + (hh - H - KV) * D + d0);
        }
    };
    const int h_start = h_first + wave + R * (int)blockIdx.y;
    f4 x[PB];
    if (h_start < nh) load(h_start, x);
    const f4 wq = *reinterpret_cast<const f4*>(a.rp.qn + d0);
    const f4 wk = *reinterpret_cast<const f4*>(a.rp.kn + d0);
    f4 cs, sn;
    rope_angles(a.rp, t, lane, cs, sn);
    for (int h0 = h_start; h0 < nh; h0 += R * (int)gridDim.y) {
        if (h0 != h_start) load(h0, x);
#pragma unroll
        for (int b = 0; b < PB; b++) {
            const int hh = h0 + PW * b;
            if (hh < nh) prep_row(a, off, t, hh, x[b], hh < H ? wq : wk, cs, sn, lane, store_kv);
        }
    }
}

struct RotateArgs {
    const float* attn;       // attention output: element t*a_ts + h*a_hs + d
    int64_t a_ts, a_hs;
    const float* gate;       // gate logits: element t*g_ts + h*g_hs + d, or null (attn is already gated)
    int64_t g_ts, g_hs;
    const float* signs;      // [H*256], +-1, indexed by e = h*256 + d
    float* xr;               // element t*x_ts + h*x_hs + d
    int64_t x_ts, x_hs;
    int T, W;                // W = H * 256, a multiple of 512
    LoraArgs lora;           // lora.R > 0: blocks y >= W / 512 compute the LoRA down projection of the gated rows
};

// Grid (T, W / 512) x one wave: block b of token t is elements 512b .. 512b+511 (heads 2b, 2b+1). Lane l holds
// elements 256 i + 4 l + c (i = 0, 1; c = 0..3) as v[4 i + c], loaded 16 bytes at a time: v = attn *
// sigmoid(gate) * sign, then the unnormalised Walsh-Hadamard transform (fwht512_wave), then x 1/sqrt(512).
// With a LoRA adapter, blocks y >= W / 512 (dynamic LDS of W floats) each stage token t's gated row and compute
// lora.rpb rows of u (gate_rotate.comp:14 LORA_ROW with EXPR = attn * sigmoid(gate)).
__global__ __launch_bounds__(64) void rotate_kernel(RotateArgs a) {
    const int t = blockIdx.x, lane = threadIdx.x;
    if ((int)blockIdx.y >= a.W / 512) {
        extern __shared__ float x_lds[];
        for (int e = 4 * lane; e < a.W; e += 256) {
            const int hd = e / D, d = e % D;
            f4 x = *reinterpret_cast<const f4*>(a.attn + t * a.a_ts + hd * a.a_hs + d);
            if (a.gate) {
                const f4 z = *reinterpret_cast<const f4*>(a.gate + t * a.g_ts + hd * a.g_hs + d);
#pragma unroll
                for (int c = 0; c < 4; c++) x[c] = gate_mul(x[c], z[c]);
            }
            *reinterpret_cast<f4*>(x_lds + e) = x;
        }
        __syncthreads();
        const int r0 = ((int)blockIdx.y - a.W / 512) * a.lora.rpb;
        lora_rows(a.lora, x_lds, a.W, t, r0, min(a.lora.R, r0 + a.lora.rpb), 0, 1, lane);
        return;
    }
    float v[8];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int hd = 2 * blockIdx.y + i, d = 4 * lane;
        f4 x = *reinterpret_cast<const f4*>(a.attn + t * a.a_ts + hd * a.a_hs + d);
        if (a.gate) {
            const f4 z = *reinterpret_cast<const f4*>(a.gate + t * a.g_ts + hd * a.g_hs + d);
#pragma unroll
            for (int c = 0; c < 4; c++) x[c] = gate_mul(x[c], z[c]);
        }
        x *= *reinterpret_cast<const f4*>(a.signs + hd * D + d);
#pragma unroll
        for (int c = 0; c < 4; c++) v[4 * i + c] = x[c];
    }
    fwht512_wave(v, lane);
#pragma unroll
    for (int i = 0; i < 2; i++)
        *reinterpret_cast<f4*>(a.xr + t * a.x_ts + (2 * blockIdx.y + i) * a.x_hs + 4 * lane) =
            f4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]} * INV_SQRT512;
}

struct NormRotateArgs {
    const float* h;          // hidden rows: element t*h_ts + e
    int64_t h_ts;
    const float* w;          // [D] RMSNorm weight
    const float* signs;      // [D], +-1
    float* xn;               // normed rows (element t*xn_ts + e), or null
    int64_t xn_ts;
    float* xr;               // rotated rows: element t*xr_ts + e
    int64_t xr_ts;
    int T, D;                // D a multiple of 512
    LoraArgs lora;           // lora.R > 0 (norm_rotate_row_kernel): blocks y >= 1 compute the LoRA down projection
};

// norm_rotate (kernels/norm_rotate.comp:10-33): xn = h * (1 / sqrt(sum h^2 / D + 1e-6)) * w, xr = FWHT-512(signs *
// xn) / sqrt(512) per 512-element block. Grid (T, D / 512) x one wave; each wave sums the squares of its whole row
// (the row is read from L2 by every block of it, which keeps the blocks independent) while its own block's 512
// elements load, in the lane layout of rotate_kernel.
__global__ __launch_bounds__(64) void norm_rotate_kernel(NormRotateArgs a) {
    const int t = blockIdx.x, lane = threadIdx.x, b = blockIdx.y;
    const float* x = a.h + t * a.h_ts;
    f4 xv[2], wv[2], sv[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int e = 512 * b + 256 * i + 4 * lane;
        xv[i] = *reinterpret_cast<const f4*>(x + e);
        wv[i] = *reinterpret_cast<const f4*>(a.w + e);
        sv[i] = *reinterpret_cast<const f4*>(a.signs + e);
    }
    float ss = 0.0f;
    for (int e = 4 * lane; e < a.D; e += 256) {
        const f4 v = *reinterpret_cast<const f4*>(x + e);
        ss = fmaf(v[0], v[0], ss);
        ss = fmaf(v[1], v[1], ss);
        ss = fmaf(v[2], v[2], ss);
        ss = fmaf(v[3], v[3], ss);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    const float r = 1.0f / sqrtf(ss / (float)a.D + 1e-6f);
    float v[8];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        f4 n;
#pragma unroll
        for (int c = 0; c < 4; c++) n[c] = (xv[i][c] * r) * wv[i][c];
        if (a.xn) *reinterpret_cast<f4*>(a.xn + t * a.xn_ts + 512 * b + 256 * i + 4 * lane) = n;
#pragma unroll
        for (int c = 0; c < 4; c++) v[4 * i + c] = n[c] * sv[i][c];
    }
    fwht512_wave(v, lane);
#pragma unroll
    for (int i = 0; i < 2; i++)
        *reinterpret_cast<f4*>(a.xr + t * a.xr_ts + 512 * b + 256 * i + 4 * lane) =
            f4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]} * INV_SQRT512;
}

// norm_rotate with one block per row, D / 512 <= 16 waves: each wave squares and sums its own 512 elements, the
// partial sums meet in LDS (wave order), so the row is read once (norm_rotate_kernel reads it D / 512 times).
// With a LoRA adapter, blocks y >= 1 (dynamic LDS of D floats) compute the same norm, stage the normed row
// (norm_rotate.comp:21 LORA_ROW with EXPR = h * r * w) and lora.rpb rows of u.
__global__ __launch_bounds__(1024) void norm_rotate_row_kernel(NormRotateArgs a) {
    __shared__ float ss_lds[16];
    extern __shared__ float x_lds[];
    const int t = blockIdx.x, lane = threadIdx.x & 63, b = threadIdx.x >> 6, nb = a.D / 512;
    const float* x = a.h + t * a.h_ts;
    f4 xv[2], wv[2], sv[2];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int e = 512 * b + 256 * i + 4 * lane;
        xv[i] = *reinterpret_cast<const f4*>(x + e);
        wv[i] = *reinterpret_cast<const f4*>(a.w + e);
        sv[i] = *reinterpret_cast<const f4*>(a.signs + e);
#pragma unroll
        for (int c = 0; c < 4; c++) ss = fmaf(xv[i][c], xv[i][c], ss);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) ss_lds[b] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int k = 0; k < nb; k++) tot += ss_lds[k];
    const float r = 1.0f / sqrtf(tot / (float)a.D + 1e-6f);
    if (blockIdx.y > 0) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            f4 n;
#pragma unroll
            for (int c = 0; c < 4; c++) n[c] = (xv[i][c] * r) * wv[i][c];
            *reinterpret_cast<f4*>(x_lds + 512 * b + 256 * i + 4 * lane) = n;
        }
        __syncthreads();
        const int r0 = ((int)blockIdx.y - 1) * a.lora.rpb;
        lora_rows(a.lora, x_lds, a.D, t, r0, min(a.lora.R, r0 + a.lora.rpb), b, nb, lane);
        return;
    }
    float v[8];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        f4 n;
#pragma unroll
        for (int c = 0; c < 4; c++) n[c] = (xv[i][c] * r) * wv[i][c];
        if (a.xn) *reinterpret_cast<f4*>(a.xn + t * a.xn_ts + 512 * b + 256 * i + 4 * lane) = n;
#pragma unroll
        for (int c = 0; c < 4; c++) v[4 * i + c] = n[c] * sv[i][c];
    }
    fwht512_wave(v, lane);
#pragma unroll
    for (int i = 0; i < 2; i++)
        *reinterpret_cast<f4*>(a.xr + t * a.xr_ts + 512 * b + 256 * i + 4 * lane) =
            f4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]} * INV_SQRT512;
}

}  // namespace bn
