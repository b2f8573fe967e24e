/*
 * bn_oracle.c - CPU restatement of the Bonsai full-attention path. TEST INFRASTRUCTURE ONLY: the
 * checker for the HIP library, never part of it (see bn_oracle.h for the list of restated functions).
 *
 * Arithmetic order follows the reference shaders (paths relative to the Glimpse-Language repository):
 *  - scores: q is scaled by 0.0625 first (attn_split.comp:22-23); lane l of a 32-lane subgroup forms
 *    dot(qa, ka) + dot(qb, kb) over dims 8l..8l+7 (attn_split.comp:28-31), then subgroupAdd.
 *  - per chunk: m = max, p = exp(s - m) written over the scores, l = lane-strided partial sums then
 *    subgroupAdd (attn_split.comp:39-46); acc[d] = sum_j p_j v_j[d] sequential in j (:48-52).
 *  - combine: M = max m_s, then sequentially over s, skipping m_s = -inf: w = exp(m_s - M),
 *    L += l_s w, a += acc_s[d] w; out = a / L (attn_combine.comp:10-20).
 *  - gate: a * (1 / (1 + exp(-z))) (gate_rotate.comp:19-22).
 * Where the shading language leaves an order implementation-defined (the subgroupAdd tree, dot() and
 * whether a*b+c contracts to fma), this file fixes one: a butterfly over lane distance 1,2,4,8,16,
 * dot() as an fma chain, and fma for every multiply-accumulate. Those choices agree with any other
 * legal one only to fp32 rounding; parity against the GPU is therefore checked to tolerance.
 *
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off; no fast-math).
 */
#include "bn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------------------------------- */
/* input generation                                                                               */

uint64_t bn_or_splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* uniform in (0, 1]: 53 random bits */
static double u53(uint64_t* s) { return ((double)(bn_or_splitmix64(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

void bn_or_normal_f32(uint64_t seed, uint64_t stream, float* out, size_t n) {
    uint64_t s = seed ^ (stream * 0xD1B54A32D192ED03ull);
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    for (; i + 1 < n; i += 2) {
        double u1 = u53(&s), u2 = u53(&s);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2));
        out[i + 1] = (float)(r * sin(two_pi * u2));
    }
    if (i < n) {
        double u1 = u53(&s), u2 = u53(&s);
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
    }
}

void bn_or_rms_rows(float* x, size_t rows, int d) {
    for (size_t r = 0; r < rows; r++) {
        float* p = x + r * (size_t)d;
        double ss = 0.0;
        for (int i = 0; i < d; i++) ss += (double)p[i] * (double)p[i];
        double inv = 1.0 / sqrt(ss / d + 1e-6);
        for (int i = 0; i < d; i++) p[i] = (float)((double)p[i] * inv);
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* fp16                                                                                           */

uint16_t bn_or_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t ax = u & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u)); /* nan, inf */
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds past 65504 -> inf */
    if (ax < 0x38800000u) {                                    /* below fp16 normal range: subnormal or 0 */
        if (ax < 0x33000000u) return (uint16_t)sign;           /* < 2^-25: rounds to zero (tie at 2^-25 -> 0) */
        uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150); units of 2^-24 -> shift by (150-e) - 24 */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u; /* rebias 127 -> 15 */
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13), rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* carry into the exponent is correct */
    return (uint16_t)(sign | q);
}

float bn_or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, u;
    if (e == 0) {
        float f = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
        memcpy(&u, &f, 4);
        u |= sign;
    } else if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void bn_or_f32_to_f16_n(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = bn_or_f32_to_f16(in[i]);
}

void bn_or_f16_to_f32_n(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = bn_or_f16_to_f32(in[i]);
}

void bn_or_append(const float* k_new, const float* v_new, uint16_t* kc, uint16_t* vc, int T, int off, int KV) {
    size_t row = (size_t)KV * BN_OR_D;
    bn_or_f32_to_f16_n(k_new, kc + (size_t)off * row, (size_t)T * row);
    bn_or_f32_to_f16_n(v_new, vc + (size_t)off * row, (size_t)T * row);
}

/* ---------------------------------------------------------------------------------------------- */
/* attention                                                                                      */

/* subgroupAdd over 32 lanes: butterfly over lane distance 1, 2, 4, 8, 16 (one fixed legal order) */
static float sg_add32(float* v) {
    for (int m = 1; m < 32; m <<= 1) {
        float t[32];
        for (int l = 0; l < 32; l++) t[l] = v[l] + v[l ^ m];
        memcpy(v, t, sizeof t);
    }
    return v[0];
}

/* GLSL dot(vec4, vec4) as an fma chain */
static float dot4(const float* a, const float* b) {
    float r = a[0] * b[0];
    r = fmaf(a[1], b[1], r);
    r = fmaf(a[2], b[2], r);
    r = fmaf(a[3], b[3], r);
    return r;
}

/* One attn_split workgroup (kv head kh, split s, query row t): writes the 4 heads' partials.
 * part layout as the reference: part[((t*H + h)*ns + s)*258 + {0: m, 1: l, 2+d: acc}]. */
static void split_unit(int kh, int s, int t, int off, int H, int KV, int chunk, int ns,
                       const float* q, int64_t q_ts, int64_t q_hs, const float* kf, const float* vf,
                       float* part, float* sc /* [4*chunk] */, int p16) {
    const int D = BN_OR_D;
    int n = off + t + 1;
    int j0 = s * chunk, j1 = n < j0 + chunk ? n : j0 + chunk;
    float* pp = part + ((size_t)(t * H + kh * 4) * ns + s) * 258;
    if (j0 >= j1) {
        for (int h = 0; h < 4; h++) {
            pp[(size_t)h * ns * 258] = -INFINITY;
            pp[(size_t)h * ns * 258 + 1] = 0.0f;
        }
        return;
    }
    float qs[4][BN_OR_D];
    for (int h = 0; h < 4; h++) {
        const float* qr = q + (int64_t)t * q_ts + (int64_t)(kh * 4 + h) * q_hs;
        for (int d = 0; d < D; d++) qs[h][d] = qr[d] * 0.0625f;
    }
    int cnt = j1 - j0;
    for (int j = j0; j < j1; j++) {
        const float* k = kf + ((size_t)j * KV + kh) * D;
        for (int h = 0; h < 4; h++) {
            float lanes[32];
            for (int l = 0; l < 32; l++)
                lanes[l] = dot4(qs[h] + 8 * l, k + 8 * l) + dot4(qs[h] + 8 * l + 4, k + 8 * l + 4);
            sc[h * chunk + (j - j0)] = sg_add32(lanes);
        }
    }
    float ml[4][2];
    for (int h = 0; h < 4; h++) {
        float* sh = sc + h * chunk;
        float m = -INFINITY;
        for (int i = 0; i < cnt; i++) m = sh[i] > m ? sh[i] : m;
        float lanes[32];
        for (int l = 0; l < 32; l++) {
            float acc = 0.0f;
            for (int i = l; i < cnt; i += 32) {
                float p = expf(sh[i] - m);
                if (p16) p = bn_or_f16_to_f32(bn_or_f32_to_f16(p)); /* perturbed variant: fp16 probabilities */
                sh[i] = p;
                acc += p;
            }
            lanes[l] = acc;
        }
        ml[h][0] = m;
        ml[h][1] = sg_add32(lanes);
    }
    for (int h = 0; h < 4; h++) {
        float* ph = pp + (size_t)h * ns * 258;
        ph[0] = ml[h][0];
        ph[1] = ml[h][1];
        float* acc = ph + 2;
        for (int d = 0; d < D; d++) acc[d] = 0.0f;
        const float* sh = sc + h * chunk;
        for (int i = 0; i < cnt; i++) {
            const float* v = vf + ((size_t)(j0 + i) * KV + kh) * D;
            float p = sh[i];
            for (int d = 0; d < D; d++) acc[d] = fmaf(p, v[d], acc[d]);
        }
    }
}

/* One attn_combine workgroup (h, t) followed by the gate of gate_rotate.comp:19-22. */
static void combine_unit(int h, int t, int H, int ns, const float* part, const float* z, int64_t z_ts,
                         int64_t z_hs, float* out, int64_t o_ts, int64_t o_hs) {
    const float* p = part + (size_t)(t * H + h) * ns * 258;
    float M = -INFINITY;
    for (int s = 0; s < ns; s++) M = p[(size_t)s * 258] > M ? p[(size_t)s * 258] : M;
    float* o = out + (int64_t)t * o_ts + (int64_t)h * o_hs;
    const float* zr = z ? z + (int64_t)t * z_ts + (int64_t)h * z_hs : NULL;
    for (int d = 0; d < BN_OR_D; d++) {
        float L = 0.0f, a = 0.0f;
        for (int s = 0; s < ns; s++) {
            float m = p[(size_t)s * 258];
            if (m == -INFINITY) continue;
            float w = expf(m - M);
            L = fmaf(p[(size_t)s * 258 + 1], w, L);
            a = fmaf(p[(size_t)s * 258 + 2 + d], w, a);
        }
        float y = a / L;
        if (zr) y = y * (1.0f / (1.0f + expf(-zr[d])));
        o[d] = y;
    }
}

static int attend_f(int T, int off, int H, int KV, int chunk, const float* q, int64_t q_ts, int64_t q_hs,
                    const float* kf, const float* vf, const float* z, int64_t z_ts, int64_t z_hs, float* out,
                    int64_t o_ts, int64_t o_hs, int nthreads, int p16) {
    if (T <= 0 || off < 0 || KV <= 0 || H != 4 * KV) return -1;
    if (chunk <= 0) chunk = T <= 16 ? 64 : 512;
    int n = off + T;
    int ns = (n + chunk - 1) / chunk;
    float* part = (float*)malloc(sizeof(float) * (size_t)T * H * ns * 258);
    if (!part) return -1;
    int units = KV * ns * T;
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float* sc = (float*)malloc(sizeof(float) * 4 * (size_t)chunk);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int u = 0; u < units; u++) {
            int kh = u % KV, s = (u / KV) % ns, t = u / (KV * ns);
            split_unit(kh, s, t, off, H, KV, chunk, ns, q, q_ts, q_hs, kf, vf, part, sc, p16);
        }
        free(sc);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int u = 0; u < H * T; u++)
            combine_unit(u % H, u / H, H, ns, part, z, z_ts, z_hs, out, o_ts, o_hs);
    }
    (void)nthreads;
    free(part);
    return 0;
}

int bn_or_attend(int T, int off, int H, int KV, int chunk, const float* q, int64_t q_ts, int64_t q_hs,
                 const uint16_t* kc, const uint16_t* vc, const float* z, int64_t z_ts, int64_t z_hs, float* out,
                 int64_t o_ts, int64_t o_hs, int nthreads) {
    return bn_or_attend_ex(T, off, H, KV, chunk, q, q_ts, q_hs, kc, vc, z, z_ts, z_hs, out, o_ts, o_hs, nthreads, 0);
}

int bn_or_attend_ex(int T, int off, int H, int KV, int chunk, const float* q, int64_t q_ts, int64_t q_hs,
                    const uint16_t* kc, const uint16_t* vc, const float* z, int64_t z_ts, int64_t z_hs, float* out,
                    int64_t o_ts, int64_t o_hs, int nthreads, int flags) {
    if (T <= 0 || off < 0 || KV <= 0 || H != 4 * KV) return -1;
    size_t n = (size_t)(off + T) * KV * BN_OR_D;
    float* kf = (float*)malloc(sizeof(float) * n);
    float* vf = (float*)malloc(sizeof(float) * n);
    if (!kf || !vf) {
        free(kf);
        free(vf);
        return -1;
    }
    bn_or_f16_to_f32_n(kc, kf, n);
    bn_or_f16_to_f32_n(vc, vf, n);
    int r = attend_f(T, off, H, KV, chunk, q, q_ts, q_hs, kf, vf, z, z_ts, z_hs, out, o_ts, o_hs, nthreads,
                     flags & BN_OR_P16);
    free(kf);
    free(vf);
    return r;
}

int bn_or_decode_ragged(int nseq, int H, int KV, int chunk, const float* q, int64_t q_ts, const uint16_t* kc,
                        const uint16_t* vc, const int64_t* kv_off, const int32_t* kv_len, const float* z,
                        int64_t z_ts, float* out, int64_t o_ts, int nthreads) {
    return bn_or_decode_ragged_ex(nseq, H, KV, chunk, q, q_ts, kc, vc, kv_off, kv_len, z, z_ts, out, o_ts, nthreads, 0);
}

int bn_or_decode_ragged_ex(int nseq, int H, int KV, int chunk, const float* q, int64_t q_ts, const uint16_t* kc,
                           const uint16_t* vc, const int64_t* kv_off, const int32_t* kv_len, const float* z,
                           int64_t z_ts, float* out, int64_t o_ts, int nthreads, int flags) {
    for (int i = 0; i < nseq; i++) {
        if (kv_len[i] < 1) return -1;
        size_t row = (size_t)KV * BN_OR_D;
        int r = bn_or_attend_ex(1, kv_len[i] - 1, H, KV, chunk, q + (int64_t)i * q_ts, q_ts, BN_OR_D,
                                kc + (size_t)kv_off[i] * row, vc + (size_t)kv_off[i] * row,
                                z ? z + (int64_t)i * z_ts : NULL, z_ts, BN_OR_D, out + (int64_t)i * o_ts, o_ts,
                                BN_OR_D, nthreads, flags);
        if (r) return r;
    }
    return 0;
}

/* ---------------------------------------------------------------------------------------------- */
/* attn_prep (attn_prep.comp:13-59)                                                               */

void bn_or_sincos(float x, float* s, float* c) {
    float k = rintf(x * 0.6366197723675814f);
    float r = fmaf(-k, 1.5707963705062866f, x);
    r = fmaf(-k, -4.371139000186241e-08f, r);
    float r2 = r * r;
    float sr = r + r * r2 * (-1.6666654611e-1f + r2 * (8.3321608736e-3f + r2 * -1.9515295891e-4f));
    float cr = 1.0f - 0.5f * r2 +
               r2 * r2 * (4.166664568298827e-2f + r2 * (-1.388731625493765e-3f + r2 * 2.443315711809948e-5f));
    int q = (int)k & 3;
    if (q == 0) { *s = sr; *c = cr; }
    else if (q == 1) { *s = cr; *c = -sr; }
    else if (q == 2) { *s = -sr; *c = -cr; }
    else { *s = -cr; *c = sr; }
}

void bn_or_prep(const float* qp, const float* kp, const float* vp, const float* qn, const float* kn,
                const int32_t* pos, const float* inv_freq, float* qout, uint16_t* kc, uint16_t* vc, int T, int off,
                int H, int KV, int ROT, int s1, int s2) {
    const int D = BN_OR_D;
    for (int t = 0; t < T; t++) {
        for (int hh = 0; hh < H + 2 * KV; hh++) {
            if (hh >= H + KV) {
                int kh = hh - H - KV;
                for (int d = 0; d < D; d++)
                    vc[((size_t)(off + t) * KV + kh) * D + d] = bn_or_f32_to_f16(vp[(size_t)t * KV * D + kh * D + d]);
                continue;
            }
            int isq = hh < H;
            const float* src = isq ? qp + (size_t)t * H * 512 + (size_t)hh * 512 : kp + (size_t)t * KV * D + (hh - H) * D;
            const float* w = isq ? qn : kn;
            float x[BN_OR_D], buf[BN_OR_D];
            float red[8];
            for (int sid = 0; sid < 8; sid++) {
                float lanes[32];
                for (int l = 0; l < 32; l++) lanes[l] = src[sid * 32 + l] * src[sid * 32 + l];
                red[sid] = sg_add32(lanes);
            }
            float lanes[32];
            for (int l = 0; l < 32; l++) lanes[l] = l < 8 ? red[l] : 0.0f;
            float r = 1.0f / sqrtf(sg_add32(lanes) / 256.0f + 1e-6f);
            for (int d = 0; d < D; d++) {
                x[d] = src[d] * r * w[d];
                buf[d] = x[d];
            }
            for (int d = 0; d < ROT && d < D; d++) {
                int half = ROT / 2, i = d % half;
                int sel = (i % 3 == 1 && i < 3 * s1) ? 1 : ((i % 3 == 2 && i < 3 * s2) ? 2 : 0);
                float ang = (float)pos[sel * T + t] * inv_freq[i];
                float sn, cs;
                bn_or_sincos(ang, &sn, &cs);
                x[d] = d < half ? x[d] * cs - buf[d + half] * sn : x[d] * cs + buf[d - half] * sn;
            }
            if (isq)
                memcpy(qout + ((size_t)t * H + hh) * D, x, sizeof x);
            else
                for (int d = 0; d < D; d++) kc[((size_t)(off + t) * KV + (hh - H)) * D + d] = bn_or_f32_to_f16(x[d]);
        }
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* gate_rotate (gate_rotate.comp:11-26; fwht512 of common.glsl:55-72)                             */

void bn_or_gate_rotate(const float* attn, const float* qp, const float* signs, float* xr, int T, int W) {
    const float inv_sqrt512 = 0.044194173824159216f;
    for (int t = 0; t < T; t++) {
        for (int b0 = 0; b0 + 512 <= W; b0 += 512) {
            float v[512];
            for (int i = 0; i < 512; i++) {
                int e = b0 + i, hd = e >> 8, d = e & 255;
                float gt = qp[(size_t)t * 2 * W + hd * 512 + 256 + d];
                float a = attn[(size_t)t * W + e];
                v[i] = (a * (1.0f / (1.0f + expf(-gt)))) * signs[e];
            }
            /* stages over index bits 0..8: the lane stages (bits 0-4) then the in-register ones (5-8) */
            for (int m = 1; m < 512; m <<= 1)
                for (int i = 0; i < 512; i++)
                    if (!(i & m)) {
                        float a = v[i], b = v[i + m];
                        v[i] = a + b;
                        v[i + m] = a - b;
                    }
            for (int i = 0; i < 512; i++) xr[(size_t)t * W + b0 + i] = v[i] * inv_sqrt512;
        }
    }
}

/* LORA_ROW (rot.glsl:19-40): in a 128-thread workgroup, thread i = 32 SID + LANE sums dot(A[row][k .. k+3],
 * x[k .. k+3]) for k = 4 i, 4 i + 512, ... in that order (dot taken left to right, products not fused), each
 * subgroup adds its 32 lanes (subgroupAdd, restated as sg_add32), then the four subgroup sums are added left to
 * right (lred[4q] + lred[4q+1] + lred[4q+2] + lred[4q+3]). */
static float lora_row(const uint16_t* a, const float* x, int K) {
    float part[4];
    for (int sid = 0; sid < 4; sid++) {
        float lanes[32];
        for (int l = 0; l < 32; l++) {
            float acc = 0.0f;
            for (int k = (sid * 32 + l) * 4; k < K; k += 512) {
                float d = bn_or_f16_to_f32(a[k]) * x[k] + bn_or_f16_to_f32(a[k + 1]) * x[k + 1];
                d = d + bn_or_f16_to_f32(a[k + 2]) * x[k + 2];
                d = d + bn_or_f16_to_f32(a[k + 3]) * x[k + 3];
                acc += d;
            }
            lanes[l] = acc;
        }
        part[sid] = sg_add32(lanes);
    }
    return ((part[0] + part[1]) + part[2]) + part[3];
}

void bn_or_lora(const uint16_t* A, const float* x, int64_t x_ts, float* u, int64_t u_ts, int T, int K, int R) {
    for (int t = 0; t < T; t++)
        for (int r = 0; r < R; r++) u[(size_t)t * u_ts + r] = lora_row(A + (size_t)r * K, x + (size_t)t * x_ts, K);
}

void bn_or_lora_gate(const uint16_t* A, const float* attn, const float* qp, float* u, int64_t u_ts, int T, int W,
                     int R) {
    float* x = (float*)malloc((size_t)W * sizeof(float));
    for (int t = 0; t < T; t++) {
        for (int e = 0; e < W; e++) {
            const int hd = e >> 8, d = e & 255;
            const float gt = qp[(size_t)t * 2 * W + hd * 512 + 256 + d];
            x[e] = attn[(size_t)t * W + e] * (1.0f / (1.0f + expf(-gt)));
        }
        for (int r = 0; r < R; r++) u[(size_t)t * u_ts + r] = lora_row(A + (size_t)r * W, x, W);
    }
    free(x);
}

/* qmm3.comp:16-40: the weight of (n, k) is ((float)code - 1.0) * scale (qmm3.comp:32, exact in fp32), each output
 * sums x * w over k in order (qmm3.comp:34-38), then store_post (qmv.glsl:10-15): y = (add ? y + v : v) +
 * lora_acc, lora_acc = sum_j u[j] * B[n][j] in j order (qmv.glsl:4-8). */
void bn_or_ternary(const uint32_t* W, const uint16_t* S, const float* X, int64_t x_ts, float* Y, int64_t y_ts,
                   int T, int K, int O, int add, const uint16_t* B, const float* U, int64_t u_ts, int lr, int nthreads) {
    const int kw = K / 16, kg = K / 128;
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
    for (int n = 0; n < O; n++) {
        float* w = (float*)malloc((size_t)K * sizeof(float));
        for (int k = 0; k < K; k++) {
            const uint32_t code = (W[(size_t)n * kw + k / 16] >> (2 * (k % 16))) & 3u;
            w[k] = ((float)code - 1.0f) * bn_or_f16_to_f32(S[(size_t)n * kg + k / 128]);
        }
        for (int t = 0; t < T; t++) {
            const float* x = X + (size_t)t * x_ts;
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc = fmaf(x[k], w[k], acc);
            float* y = Y + (size_t)t * y_ts + n;
            float yv = add ? *y + acc : acc;
            if (B && lr > 0) {
                float la = 0.0f;
                for (int j = 0; j < lr; j++) la = fmaf(U[(size_t)t * u_ts + j], bn_or_f16_to_f32(B[(size_t)n * lr + j]), la);
                yv = yv + la;
            }
            *y = yv;
        }
        free(w);
    }
}

/* norm_rotate.comp:10-33. The sum of squares follows rot.glsl:4-18 (row_ss): 16 partial sums, partial g holding
 * elements i0 + 32 g + lane of every 512-block i0 per lane (fp32, in i0 order), each summed over its 32 lanes, then
 * the 16 partials; r = 1 / sqrt(ss / D + EPS) with EPS = 1e-6 (common.glsl); a = (x * r) * w; v = a * sign, the
 * 512-point FWHT in stage order over index bits 0..8, xr = v * 1/sqrt(512). */
void bn_or_norm_rotate(const float* h, const float* w, const float* signs, float* xn, float* xr, int T, int D) {
    const float inv_sqrt512 = 0.044194173824159216f;
    for (int t = 0; t < T; t++) {
        const float* x = h + (size_t)t * D;
        float part[16];
        for (int g = 0; g < 16; g++) {
            float lanes[32];
            for (int l = 0; l < 32; l++) {
                float acc = 0.0f;
                for (int i0 = 0; i0 < D; i0 += 512) {
                    float v = x[i0 + 32 * g + l];
                    acc += v * v;
                }
                lanes[l] = acc;
            }
            part[g] = sg_add32(lanes);
        }
        float ss = 0.0f;
        for (int g = 0; g < 16; g++) ss += part[g];
        const float r = 1.0f / sqrtf(ss / (float)D + 1e-6f);
        for (int b0 = 0; b0 < D; b0 += 512) {
            float v[512];
            for (int i = 0; i < 512; i++) {
                float a = (x[b0 + i] * r) * w[b0 + i];
                if (xn) xn[(size_t)t * D + b0 + i] = a;
                v[i] = a * signs[b0 + i];
            }
            for (int m = 1; m < 512; m <<= 1)
                for (int i = 0; i < 512; i++)
                    if (!(i & m)) {
                        float a = v[i], b = v[i + m];
                        v[i] = a + b;
                        v[i + m] = a - b;
                    }
            for (int i = 0; i < 512; i++) xr[(size_t)t * D + b0 + i] = v[i] * inv_sqrt512;
        }
    }
}
