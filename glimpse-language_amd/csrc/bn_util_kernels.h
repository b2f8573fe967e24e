// Small kernels around the attention call: cache append and workspace fill.
#pragma once
#include "bn_device.h"

namespace bn {

// Cache rows [off, off+T) <- fp16(k_new), fp16(v_new); attn_prep.comp:36-39,58 with fp16 storage.
// n8 = T*KV*256/8 groups of 8 elements; row = KV*256 elements per cache row; off = call_off(dyn, off_max).
__global__ __launch_bounds__(256) void append_kernel(const float* __restrict__ kn, const float* __restrict__ vn,
                                                     uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                     int64_t row, int off_max, const uint32_t* dyn, int64_t n8) {
    asm volatile("" ::"s"(kn), "s"(vn), "s"(kc), "s"(vc), "s"(row), "s"(n8));  // argument words in one round trip
    const int64_t o = (int64_t)call_off(dyn, off_max) * row;
    if (dyn_over(dyn, off_max)) return;  // an offset past the bound appends nothing (the flag is set)
    uint16_t* kdst = kc + o;
    uint16_t* vdst = vc + o;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
        st_h8(kdst + i * 8, ld_f32x8_as_h8(kn + i * 8));
        st_h8(vdst + i * 8, ld_f32x8_as_h8(vn + i * 8));
    }
}

// Prefix snapshot copy (mod.rs:211-244 encode_copy_state, KV part): rows [0, len) of every layer of the K and the V
// cache into another state's caches, both caches in one launch. The copy is cut into chunks of KVC_U x 256
// consecutive 16-byte groups of one layer's w16 (the used rows are contiguous in a layer), cpl chunks per layer;
// block t copies chunk t, of cache t / cpl / n_layers and layer t / cpl % n_layers. A thread's KVC_U loads are all
// in flight before its stores, a wave's load or store instruction covers 1 KB contiguous, and the stores are
// non-temporal: the snapshot is not read back soon, and streaming it past the caches measured 5-30% faster than
// ordinary stores. Layer pitches sp16 / dp16 in 16-byte groups (cap * KV * 256 * 2 / 16 of each state).
constexpr int KVC_U = 4;
__global__ __launch_bounds__(256) void kv_copy_kernel(const u4* __restrict__ sk, const u4* __restrict__ sv,
                                                      u4* __restrict__ dk, u4* __restrict__ dv, int64_t w16,
                                                      int64_t sp16, int64_t dp16, int n_layers, int cpl) {
    const int t = blockIdx.x, y = t / cpl, c = y >= n_layers, layer = c ? y - n_layers : y;
    const u4* src = (c ? sv : sk) + (int64_t)layer * sp16;
    u4* dst = (c ? dv : dk) + (int64_t)layer * dp16;
    const int64_t i0 = (int64_t)(t - y * cpl) * (256 * KVC_U) + threadIdx.x;
    u4 v[KVC_U];
#pragma unroll
    for (int u = 0; u < KVC_U; u++)
        if (i0 + 256 * u < w16) v[u] = src[i0 + 256 * u];
#pragma unroll
    for (int u = 0; u < KVC_U; u++)
        if (i0 + 256 * u < w16) __builtin_nontemporal_store(v[u], dst + i0 + 256 * u);
}

// Zero fill with vector stores (no memset node, so it is safe to capture in a graph).
__global__ __launch_bounds__(256) void fill_zero_kernel(u4* p, int64_t n16, uint8_t* tail, int ntail) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t i = i0; i < n16; i += stride) p[i] = u4{0u, 0u, 0u, 0u};
    if (i0 < ntail) tail[i0] = 0;
}

}  // namespace bn
