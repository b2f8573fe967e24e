// The steps either side of the attention product: attn_prep (q/k RMS-norm, interleaved mRoPE, fp16 K/V append)
// before it and gate_rotate (sigmoid gate, sign flip, 512-point Walsh-Hadamard transform) after it.
//
// Semantics follow kernels/attn_prep.comp:29-59 and kernels/gate_rotate.comp:11-26 with fwht512 of
// kernels/common.glsl:55-72 in the reference; the decompositions are this file's own (one wave per head row,
// reductions and butterflies across the wave with lane shuffles, no LDS).
#pragma once
#include "bn_device.h"

namespace bn {

struct PrepArgs {
    const float* qp;         // q rows: element t*qp_ts + h*qp_hs + d (the q half of the q_proj output)
    int64_t qp_ts, qp_hs;
    const float* kp;         // [T][KV][256]
    const float* vp;         // [T][KV][256]
    const float* qn;         // [256] q norm weight
    const float* kn;         // [256] k norm weight
    const int32_t* pos;      // [3][T] mRoPE positions (t, h, w rows)
    const float* inv_freq;   // [rot / 2]
    float* q;                // element t*q_ts + h*q_hs + d: fp32 ...
    uint16_t* q16;           // ... or fp16 bits when non-null
    int64_t q_ts, q_hs;
    uint16_t* kc;            // fp16 [cap][KV][256]: rows off .. off+T-1 written
    uint16_t* vc;
    int T, off, H, KV, rot, s1, s2;
};

// Grid (T, ceil((H + 2 KV) / 4)) x 4 waves; wave = one head row: q heads [0, H), k heads [H, H+KV), v heads
// [H+KV, H+2KV). Lane l holds dims 4l .. 4l+3.
//   q/k: x * (1 / sqrt(sum x^2 / 256 + 1e-6)) * w (a wave-wide sum), then on dims d < rot (pairs d, d + rot/2;
//   pair index i = d mod rot/2): position row sel = 1 if i % 3 == 1 and i < 3 s1, 2 if i % 3 == 2 and i < 3 s2,
//   else 0; angle pos[sel][t] * inv_freq[i]; x' = x cos - x[d + rot/2] sin (first half), x cos + x[d - rot/2]
//   sin (second half). The partner element is held by lane l +- rot/8.
//   v: copied. k and v are rounded to fp16 (nearest even) into cache row off + t.
__global__ __launch_bounds__(256) void prep_kernel(PrepArgs a) {
    const int t = blockIdx.x, lane = threadIdx.x & 63;
    const int hh = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int H = a.H, KV = a.KV, d0 = 4 * lane;
    if (hh >= H + 2 * KV) return;
    const int64_t kvd = (int64_t)KV * D;
    if (hh >= H + KV) {
        const int kh = hh - H - KV;
        const f4 v = *reinterpret_cast<const f4*>(a.vp + t * kvd + kh * D + d0);
        const h4 y = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        *reinterpret_cast<h4*>(a.vc + ((int64_t)(a.off + t) * KV + kh) * D + d0) = y;
        return;
    }
    const bool isq = hh < H;
    f4 x = isq ? *reinterpret_cast<const f4*>(a.qp + t * a.qp_ts + hh * a.qp_hs + d0)
               : *reinterpret_cast<const f4*>(a.kp + t * kvd + (hh - H) * D + d0);
    float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
    const float r = 1.0f / sqrtf(ss / 256.0f + 1e-6f);
    const f4 w = *reinterpret_cast<const f4*>((isq ? a.qn : a.kn) + d0);
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = x[e] * r * w[e];
    const int half = a.rot >> 1;
    if (d0 < a.rot) {
        // partner dims d -+ half are in lane l -+ half/4 (rot is a multiple of 8, so a lane's four dims sit on
        // one side of `half`); the partner lanes are all inside this branch
        const int pl = d0 < half ? lane + (half >> 2) : lane - (half >> 2);
        f4 xp;
#pragma unroll
        for (int e = 0; e < 4; e++) xp[e] = __shfl(x[e], pl);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int d = d0 + e, i = d % half;
            const int sel = (i % 3 == 1 && i < 3 * a.s1) ? 1 : ((i % 3 == 2 && i < 3 * a.s2) ? 2 : 0);
            const float ang = (float)a.pos[sel * a.T + t] * a.inv_freq[i];
            float sn, cs;
            sincosf(ang, &sn, &cs);
            x[e] = d < half ? x[e] * cs - xp[e] * sn : x[e] * cs + xp[e] * sn;
        }
    }
    if (isq) {
        if (a.q16) {
            const h4 y = {(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
            *reinterpret_cast<h4*>(a.q16 + t * a.q_ts + hh * a.q_hs + d0) = y;
        } else {
            *reinterpret_cast<f4*>(a.q + t * a.q_ts + hh * a.q_hs + d0) = x;
        }
    } else {
        const h4 y = {(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
        *reinterpret_cast<h4*>(a.kc + ((int64_t)(a.off + t) * KV + (hh - H)) * D + d0) = y;
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
};

// Grid (T, W / 512) x one wave: block b of token t is elements 512b .. 512b+511 (two heads). Lane l holds elements
// l + 64e (e = 0..7): v = attn * sigmoid(gate) * sign, then the unnormalised Walsh-Hadamard transform
// (fwht512_wave), then x 1/sqrt(512).
__global__ __launch_bounds__(64) void rotate_kernel(RotateArgs a) {
    const int t = blockIdx.x, b0 = blockIdx.y * 512, lane = threadIdx.x;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int i = b0 + lane + 64 * e, hd = i >> 8, d = i & 255;
        const float at = a.attn[t * a.a_ts + hd * a.a_hs + d];
        v[e] = (a.gate ? gate_mul(at, a.gate[t * a.g_ts + hd * a.g_hs + d]) : at) * a.signs[i];
    }
    fwht512_wave(v, lane);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int i = b0 + lane + 64 * e;
        a.xr[t * a.x_ts + (i >> 8) * a.x_hs + (i & 255)] = v[e] * INV_SQRT512;
    }
}

}  // namespace bn
