// Device-side helpers shared by the attention kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bn {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr int D = 256;                       // head dim (fixed by the architecture)
constexpr float LOG2E = 1.44269504088896340736f;
constexpr float QK_SCALE = 0.0625f;          // 1/sqrt(256), exact

// 16 bytes of fp16 at p (16-byte aligned)
__device__ __forceinline__ h8 ld_h8(const uint16_t* p) {
    return __builtin_bit_cast(h8, *reinterpret_cast<const u4*>(p));
}
// the same, non-temporal: for K/V rows streamed once (measured on MI355X: ~6.8 TB/s read ceiling with
// non-temporal loads against ~6.2 TB/s with default loads)
__device__ __forceinline__ h8 ld_h8_nt(const uint16_t* p) {
    return __builtin_bit_cast(h8, __builtin_nontemporal_load(reinterpret_cast<const u4*>(p)));
}
__device__ __forceinline__ void st_h8(uint16_t* p, h8 v) {
    *reinterpret_cast<u4*>(p) = __builtin_bit_cast(u4, v);
}
// 8 fp32 at p (16-byte aligned) rounded to fp16, nearest even (v_cvt_f16_f32)
__device__ __forceinline__ h8 ld_f32x8_as_h8(const float* p) {
    f4 a = *reinterpret_cast<const f4*>(p);
    f4 b = *reinterpret_cast<const f4*>(p + 4);
    h8 r;
    r[0] = (_Float16)a[0]; r[1] = (_Float16)a[1]; r[2] = (_Float16)a[2]; r[3] = (_Float16)a[3];
    r[4] = (_Float16)b[0]; r[5] = (_Float16)b[1]; r[6] = (_Float16)b[2]; r[7] = (_Float16)b[3];
    return r;
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x mfma32(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// x from lane l and lane l ^ 32 (v_permlane32_swap: no LDS round trip), combined
__device__ __forceinline__ float max_xhalf(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xhalf(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Set (to 1) by any kernel that finds a device offset above its call's host bound; kernels never clear it. The host
// reads and clears it with bn_dyn_overflow. One copy per device, from the library's load until the process ends.
__device__ unsigned int dyn_overflow;

// The device offset at dyn lies above the host bound off_max: the call's cache appends are skipped.
__device__ __forceinline__ bool dyn_over(const uint32_t* dyn, int off_max) {
    return dyn != nullptr && *dyn > (uint32_t)off_max;
}

// The cache offset of a call: the host value, or (graph replay) the device value at dyn. A device value above the
// host value (which sizes the launch) is taken as the host value, and the overflow flag is set (a vector atomic).
__device__ __forceinline__ int call_off(const uint32_t* dyn, int off_max) {
    if (!dyn) return off_max;
    const uint32_t d = *dyn;
    if (d <= (uint32_t)off_max) return (int)d;
    __hip_atomic_fetch_or(&dyn_overflow, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return off_max;
}

// reference gate: a * (1 / (1 + exp(-z)))  (gate_rotate.comp:19-22)
__device__ __forceinline__ float gate_mul(float a, float z) { return a * (1.0f / (1.0f + expf(-z))); }
// the same product on v_exp_f32 / v_rcp_f32 (about 2 ulp): for epilogues that gate many rows per lane
__device__ __forceinline__ float gate_mul_fast(float a, float z) {
    return a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * LOG2E));
}

// x from lane (lane ^ m) for the DPP controls used below: 0xB1 quad_perm [1,0,3,2] (m = 1), 0x4E quad_perm
// [2,3,0,1] (m = 2), 0x1B quad_perm [3,2,1,0] (m = 3), 0x141 row_half_mirror (m = 7 inside each 8 lanes), 0x128
// row_ror:8 (m = 8 inside each row of 16)
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Unnormalised 512-point Walsh-Hadamard transform of v held by one wave: 6 index bits are lane bits, 3 are bits
// of e (v[e], e = 0..7); which index bits they are is the caller's mapping (the callers here use element
// 256 (e/4) + 4 lane + e%4, so a lane's values are two 16-byte groups). H_512 is the tensor product of H_2 over
// the 9 bits, so any such mapping and any stage order give H_512 v (common.glsl:55-72 fwht512 computes the same
// transform with 32-lane subgroups and 16 elements per lane). A cross-lane butterfly pairs lane l with l ^ m:
// the lower lane needs own + partner, the upper one partner - own. Every lane computes own + s partner instead
// (s = -1 on the upper lane), which leaves the upper lane's result negated; the two lanes of a later stage have
// taken the same sides so far, so they carry the same sign, and the signs are settled once at the end:
// (-1)^popcount(l). The partners come from DPP moves (m = 1, 2, 4 = 7 then 3, 8) and v_permlane16/32_swap
// (m = 16, 32), with no LDS traffic.
__device__ __forceinline__ void fwht512_wave(float (&v)[8], int lane) {
    const float s1 = (lane & 1) ? -1.0f : 1.0f, s2 = (lane & 2) ? -1.0f : 1.0f, s4 = (lane & 4) ? -1.0f : 1.0f;
    const float s8 = (lane & 8) ? -1.0f : 1.0f, s16 = (lane & 16) ? -1.0f : 1.0f, s32 = (lane & 32) ? -1.0f : 1.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = fmaf(dpp_f32<0xB1>(v[e]), s1, v[e]);
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = fmaf(dpp_f32<0x4E>(v[e]), s2, v[e]);
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = fmaf(dpp_f32<0x1B>(dpp_f32<0x141>(v[e])), s4, v[e]);
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = fmaf(dpp_f32<0x128>(v[e]), s8, v[e]);
    // permlane16_swap(x, x): first result = rows (0, 0, 2, 2) of x, second = rows (1, 1, 3, 3); own + s partner
    // is then first * s + second on either side
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[e]), __float_as_uint(v[e]), false, false);
        v[e] = fmaf(__uint_as_float(r[0]), s16, __uint_as_float(r[1]));
    }
    // permlane32_swap(x, x): first = lanes 0-31 of x in both halves, second = lanes 32-63
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[e]), __float_as_uint(v[e]), false, false);
        v[e] = fmaf(__uint_as_float(r[0]), s32, __uint_as_float(r[1]));
    }
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int e = 0; e < 8; e++)
            if ((e & h) == 0) {
                const float p = v[e], q = v[e + h];
                v[e] = p + q;
                v[e + h] = p - q;
            }
    const float sg = (__builtin_popcount(lane & 63) & 1) ? -1.0f : 1.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] *= sg;
}

constexpr float INV_SQRT512 = 0.044194173824159216f;

// The rotated output of one head pair: `lds` holds y[i*256 + d] * sign for heads 2j + i (i = 0, 1); the calling
// wave transforms the 512 elements and stores them at o (head 2j) with head stride o_hs (a multiple of 4, o
// 16-byte aligned). All 64 lanes take part.
__device__ __forceinline__ void rotate_pair_store(const float* lds, float* o, int64_t o_hs, int lane) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const f4 x = *reinterpret_cast<const f4*>(lds + 256 * i + 4 * lane);
#pragma unroll
        for (int c = 0; c < 4; c++) v[4 * i + c] = x[c];
    }
    fwht512_wave(v, lane);
#pragma unroll
    for (int i = 0; i < 2; i++)
        *reinterpret_cast<f4*>(o + i * o_hs + 4 * lane) =
            f4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]} * INV_SQRT512;
}

// The same for block j of one (row, kv head) group: `lds` holds the group's 4 heads, o is the group's head 0.
__device__ __forceinline__ void rotate_group_store(const float* lds, float* o, int64_t o_hs, int j, int lane) {
    rotate_pair_store(lds + j * 512, o + 2 * j * o_hs, o_hs, lane);
}

// x *= s with x held in an accumulation register: O stays in the accumulation registers for the whole loop (a plain
// multiply makes the compiler keep two copies of O and move all 128 registers at every tile)
__device__ __forceinline__ void scale_acc(float& x, float s) {
    float t;
    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                 : "+a"(x), "=&v"(t)
                 : "v"(s));
}


}  // namespace bn
