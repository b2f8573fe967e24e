/*
 * bonsai_attn.h - C ABI of the MI355X (gfx950) full-attention path of the Bonsai runtime.
 *
 * One call replaces the attention arm of the runtime's layer encoder
 * (src/bonsai/runtime/model.rs:815-894 in the Glimpse-Language repository), which dispatches
 *     attn_prep     -> K/V rows appended to the cache at [off, off + T)   (kernels/attn_prep.comp:36-39,58)
 *     attn_split    -> split-K causal GQA partials                          (kernels/attn_split.comp:9-58)
 *     attn_combine  -> log-sum-exp merge of the splits                      (kernels/attn_combine.comp:6-21)
 *     gate_rotate   -> a * sigmoid(gate), and with `signs` the Hadamard     (kernels/gate_rotate.comp:19-25)
 *                      rotation that makes o_proj's input
 * through Cmd::run (src/bonsai/runtime/gpu_vk.rs:843-882, gpu.rs:169-255). Query/key normalisation and
 * rotary embedding (the rest of attn_prep) happen before the call: q and k_new arrive post-norm, post-RoPE,
 * or go through bn_attn_prep first.
 *
 * Conventions
 *   - head_dim is 256 and H == 4 * KV (the runtime's fixed GQA 4:1, model.rs:89-129).
 *   - Query row t sits at position off + t and attends to cache rows [0, off + t + 1) of kv head h / 4
 *     (causal, including itself and, for several rows, causal among them: attn_split.comp:15).
 *   - The KV cache is fp16 (IEEE binary16 bits in uint16_t), row-major [cap][KV][256]: element
 *     ((pos * KV + kh) * 256 + d). The reference stores fp32 in the same position-major layout
 *     (model.rs:255-267); rows of one prefix stay one contiguous range.
 *   - k_new / v_new (fp32 [T][KV][256], dense) are rounded to fp16 (nearest even) and written to cache rows
 *     [off, off + T) by the call. Pass both NULL when those rows are already in the cache.
 *   - Strides are in elements. Tensors of different calls may alias only as stated.
 *   - Every call is ordered on `stream` (a hipStream_t; NULL = the default stream), returns without a host
 *     synchronisation, and allocates nothing: device memory (cache, inputs, outputs, workspace) belongs to
 *     the caller.
 *   - A bn_ctx may be used from several threads only if the caller serialises the calls, as the runtime
 *     does behind its model mutex (src/bonsai/handle.rs:96-103).
 *   - Errors are status codes; nothing is thrown across the ABI. Argument checks run on the host before any
 *     launch, so a rejected call has no effect on the device.
 */
#ifndef BONSAI_ATTN_H
#define BONSAI_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BN_HEAD_DIM 256
#define BN_ABI_VERSION 6

typedef enum bn_status {
    BN_OK = 0,
    BN_EINVAL = 1,  /* bad shape, pointer, stride or ratio (replaces the reference's shape asserts, model.rs:671-672) */
    BN_ENOWS = 2,   /* workspace missing or smaller than the size query returned */
    BN_ELAUNCH = 3, /* a kernel launch failed (replaces `expect("GPU error")`, gpu_vk.rs:1144) */
    BN_EDEVICE = 4, /* no usable gfx950 device / HIP runtime error at context creation */
} bn_status;

typedef struct bn_ctx bn_ctx;
typedef void* bn_stream; /* hipStream_t */

/* One attention layer call for T query rows of one sequence. */
typedef struct bn_attn_args {
    uint32_t T;   /* query rows (1 = decode step, 2..16 = speculative verify, more = prefill) */
    uint32_t off; /* cache rows before the first query row (the reference's state.len, model.rs:680-681) */
    uint32_t H;   /* query heads; H == 4 * KV */
    uint32_t KV;  /* kv heads */
    uint32_t cap; /* rows allocated in kc / vc; off + T <= cap */
    uint32_t flags; /* BN_Q_F16: q holds fp16 bits instead of fp32. Every kernel keeps an fp32 q's precision
                       (the MFMA ones multiply it as an fp16 hi/lo pair: a long prefill then costs about 1.5x its
                       fp16-q time, a short one about 1.1x) */

    const void* q; /* [T][H][256] query rows, post-norm and post-RoPE */
    int64_t q_ts, q_hs; /* token and head strides of q */

    const float* k_new; /* [T][KV][256] fp32, or NULL (rows already cached) */
    const float* v_new;
    uint16_t* kc; /* [cap][KV][256] fp16 cache of this layer */
    uint16_t* vc;

    const float* gate; /* sigmoid-gate logits, element t*g_ts + h*g_hs + d; NULL = no gate */
    int64_t g_ts, g_hs; /* the runtime's q_proj output [T][H][512] is used in place: gate = qp + 256,
                           g_ts = 512 * H, g_hs = 512 (gate_rotate.comp:19-20) */

    float* out;         /* [T][H][256] fp32 gated attention output (rotated when `signs` is set) */
    int64_t o_ts, o_hs;

    void* ws;        /* device workspace (split partials; for bn_attn_layer with 2..16 rows also their q),
                        >= bn_attn_workspace_size(args) bytes, 16-byte
                        aligned; NULL when the size is 0. No initialisation is needed and nothing in it
                        outlives the call. Calls that overlap in time on one workspace race. */
    size_t ws_bytes;

    const float* signs; /* [H * 256] +1/-1 (16-byte aligned), or NULL. When set, `out` receives o_proj's input
                           instead of the gated output: the rest of gate_rotate (gate_rotate.comp:22-25), i.e.
                           per row and block of 512 elements (heads 2j, 2j+1), H_512 (gated * signs) / sqrt(512).
                           The attention kernels rotate in their epilogue (the fallback prefill kernel for
                           calls too small to fill the GPU rotates in place after it). */

    const uint32_t* dyn; /* NULL, or device memory holding this call's cache offset (the reference's dynamic
                            parameter slot for replayed command buffers: attn_split.comp:12-14, attn_prep.comp:32-33,
                            filled per step by gpu_vk.rs:1035-1049). The kernels read dyn[0] when they run and use
                            it in place of `off` (the rows' positions, the keys they see, the cache rows written);
                            `off` is then the largest offset the call may see, and sizes the launch and the
                            workspace. A call captured in a HIP graph thus replays at any offset up to `off`: the
                            caller advances dyn[0] on the device between replays. A device value above `off` is an
                            error the kernels cannot return: they attend as if it were `off`, append no row (the
                            cache is left as it was), and set the device's overflow flag (bn_dyn_overflow). */

    /* LoRA down projection of the gated output (the extra rows gate_rotate computes, gate_rotate.comp:14,
     * rot.glsl:19-40, sized by rot_lora model.rs:444-454): u[t][r] = sum_e A[r][e] y[t][e], with y the gated
     * output row before the signs and the rotation (e = h * 256 + d). Computed after the attention by one more
     * launch, from `out` (undoing the rotation when `signs` is set). lora_r == 0: none. */
    const uint16_t* lora_a; /* [lora_r][H * 256] fp16, 16-byte aligned; H * 256 <= 16384 */
    float* lora_u;          /* out: u[t][r] at lora_u + t * lora_us + r */
    int64_t lora_us;
    uint32_t lora_r;
} bn_attn_args;

#define BN_Q_F16 1u

/* A batch of single-token decodes over sequences of different lengths (one new token each). */
typedef struct bn_ragged_args {
    uint32_t nseq;
    uint32_t H, KV;
    uint32_t max_len;    /* host-side upper bound of kv_len[i]; sizes the launch */
    const float* q;      /* [nseq][H][256] fp32 */
    int64_t q_ss, q_hs;  /* sequence and head strides */
    const float* k_new;  /* [nseq][KV][256] fp32 appended at row kv_off[i] + kv_len[i] - 1, or NULL */
    const float* v_new;
    uint16_t* kc;        /* fp16 rows of all sequences, [rows][KV][256] */
    uint16_t* vc;
    const int64_t* kv_off; /* device [nseq]: first cache row of sequence i */
    const int32_t* kv_len; /* device [nseq]: keys attended by sequence i including the new one, 1..max_len */
    const float* gate;   /* element i*g_ss + h*g_hs + d, or NULL */
    int64_t g_ss, g_hs;
    float* out;          /* element i*o_ss + h*o_hs + d */
    int64_t o_ss, o_hs;
    void* ws;
    size_t ws_bytes;
    const float* signs;  /* as bn_attn_args.signs */
} bn_ragged_args;

/* The step before attention for T rows (kernels/attn_prep.comp:29-59, dispatched at model.rs:828-851):
 *   q = rope(rmsnorm(qp) * q_norm), k = rope(rmsnorm(kp) * k_norm), v = vp;
 *   rmsnorm(x) = x / sqrt(mean(x^2) + 1e-6) over the 256 dims of one head (common.glsl EPS);
 *   rope: interleaved mRoPE on dims d < rot, pairs (d, d + rot/2) with pair index i = d mod rot/2 turned by
 *   angle pos[sel][t] * inv_freq[i], sel = 1 if i % 3 == 1 and i < 3*s1, 2 if i % 3 == 2 and i < 3*s2, else 0;
 *   x'[d] = x[d] cos - x[d + rot/2] sin (d < rot/2), x[d] cos + x[d - rot/2] sin (rot/2 <= d < rot).
 * k and v are rounded to fp16 (nearest even) into cache rows [off, off + T); q goes to `q` (fp32, or fp16 bits
 * with BN_Q_F16, the form the attention call takes with the same flag). The reference keeps the cache in fp32. */
typedef struct bn_prep_args {
    uint32_t T, off, H, KV, cap; /* as bn_attn_args; H == 4 * KV */
    uint32_t flags;              /* BN_Q_F16: write q as fp16 bits */
    uint32_t rot;                /* rotary dims: a multiple of 8, at most 256 (the runtime's 64) */
    uint32_t s1, s2;             /* mRoPE sections of the h and w position rows (the runtime's 11, 11) */
    const float* qp;             /* query rows before the norm: element t*qp_ts + h*qp_hs + d. The runtime's q_proj
                                    output [T][H][512] is used in place: qp_ts = 512 H, qp_hs = 512 */
    int64_t qp_ts, qp_hs;
    const float* kp;             /* [T][KV][256] k_proj output */
    const float* vp;             /* [T][KV][256] v_proj output */
    const float* q_norm;         /* [256] */
    const float* k_norm;         /* [256] */
    const int32_t* pos;          /* device [3][T]: the t, h and w position rows (unused when rot == 0) */
    const float* inv_freq;       /* device [rot / 2] */
    void* q;                     /* out: element t*q_ts + h*q_hs + d. May be qp itself with the same strides
                                    (fp32): every row is read before it is written */
    int64_t q_ts, q_hs;
    uint16_t* kc;                /* [cap][KV][256] fp16 caches; rows [off, off + T) are written */
    uint16_t* vc;
    const uint32_t* dyn;         /* as bn_attn_args.dyn: NULL, or the device offset read at run time (off its bound);
                                    the positions come from `pos`, which is device memory already */
} bn_prep_args;

/* The step after attention (kernels/gate_rotate.comp:11-26, dispatched at model.rs:878-893) without its LoRA-A
 * rows: for each row t and each block of 512 elements (two heads, e = h*256 + d),
 *   v[e] = attn[e] * sigmoid(gate[h][d]) * signs[e],   xr = H_512 v / sqrt(512)
 * with H_512 the Walsh-Hadamard matrix (common.glsl:55-72 fwht512). With gate == NULL attn is taken as already
 * gated (bn_attn_forward with a gate). */
typedef struct bn_rotate_args {   /* pointers 16-byte aligned, strides multiples of 4 elements */
    uint32_t T, H;               /* rows and heads; H even (W = 256 H elements per row) */
    const float* attn;           /* element t*a_ts + e */
    int64_t a_ts;
    const float* gate;           /* element t*g_ts + h*g_hs + d, or NULL; the q_proj output in place:
                                    gate = qp + 256, g_ts = 512 H, g_hs = 512 */
    int64_t g_ts, g_hs;
    const float* signs;          /* [W], +1 or -1 */
    float* xr;                   /* out: element t*x_ts + e; may be attn itself with the same stride */
    int64_t x_ts;
    /* the LoRA-A rows of gate_rotate (gate_rotate.comp:14, rot.glsl:19-40): u[t][r] = sum_e A[r][e] *
     * attn[t][e] * sigmoid(gate[t][e]) (the gated row before the signs), in extra blocks of the same launch */
    const uint16_t* lora_a;      /* [lora_r][W] fp16, 16-byte aligned, W <= 16384; NULL with lora_r == 0 */
    float* lora_u;               /* out: u[t][r] at lora_u + t * lora_us + r. With lora_r > 0, xr may not be attn (the
                                    LoRA blocks read attn while the rotation blocks write xr) */
    int64_t lora_us;
    uint32_t lora_r;
} bn_rotate_args;

/* The attention layers' part of a prefix-state snapshot (the reference's State: model.rs:174-186, 255-267; copied
 * by encode_copy_state, model.rs:1072-1086; saved and loaded with state_parts, model.rs:1088-1099, by
 * save_prefix / load_prefix, mod.rs:492-578): the used rows [0, len) of every attention layer's fp16 cache. */
typedef struct bn_kv_state {
    uint16_t* kc;                /* n_layers caches of cap rows each, [n_layers][cap][KV][256] fp16: layer i at */
    uint16_t* vc;                /* kc + i * cap * KV * 256 (the reference's kc/vc buffers, in fp16) */
    uint32_t n_layers, KV, cap;
    uint32_t len;                /* rows in use, <= cap */
} bn_kv_state;

/* The KV section of a saved prefix file, little endian: the 8 bytes "BNKVF16\0", u32 version (1), u32 n_layers,
 * u32 kv_width (KV * 256), u32 len, then rows [0, len) of every layer's K cache (fp16, layer after layer), then
 * the same of V. The reference's file (magic BNSPFX01) holds the same rows in fp32 after its GDN and conv state;
 * a runtime that keeps fp16 caches writes this section in their place and bumps its own magic. */
#define BN_KV_SECTION_MAGIC "BNKVF16"
#define BN_KV_SECTION_VERSION 1u
#define BN_KV_SECTION_HEADER 24

/* A ternary packed linear (kernels/qmv.glsl:1-2; model.rs:133-139 Lin): row n of W is k / 16 uint32 words, word j
 * holding the codes of columns 16j + e at bits [2e, 2e + 2); one fp16 scale per 128 columns at s[n * k/128 + c/128];
 * the weight of column c is scale * (code - 1). */
typedef struct bn_ternary_mat {
    const uint32_t* w;       /* [o][k / 16], 16-byte aligned */
    const uint16_t* s;       /* [o][k / 128] fp16 */
    float* y;                /* output: token t's o values at y + t * y_ts */
    const uint16_t* lora_b;  /* LoRA up projection B [o][lora_r] fp16 (alpha / r folded in, lora.rs:140-146), or
                              * NULL: no adapter on this matrix (the reference's zero B) */
    uint32_t o;              /* rows: a multiple of 64 */
    int64_t y_ts;
} bn_ternary_mat;

/* Up to three matmuls sharing one input (the q/k/v projections of an attention layer; o_proj alone with
 * add = 1): y_i[t] (+)= x[t] W_i^T, then + lora_b_i . u (model.rs:455-596 qmm_lora / qmm / qmm_multi). */
typedef struct bn_ternary_args {
    uint32_t T;              /* tokens (1 = decode step, 2..16 = verify rows, more = prefill) */
    uint32_t k;              /* input width: a multiple of 128 */
    const float* x;          /* token t at x + t * x_ts (16-byte aligned, x_ts a multiple of 4) */
    int64_t x_ts;
    uint32_t n_mats;         /* 1..3 */
    uint32_t add;            /* 1: y += result (o_proj into the residual stream, model.rs:893) */
    bn_ternary_mat mat[3];
    const float* lora_u;     /* LoRA down projections: token t, matrix i at lora_u + t * lora_us + i * lora_r */
    int64_t lora_us;
    uint32_t lora_r;         /* LoRA rank (0: none) */
    void* work;              /* T > 32: optional device workspace of bn_ternary_workspace_size(T, k) bytes, 256-byte
                              * aligned, in which x is split once per call (faster); NULL: every block of the GEMM
                              * splits its own x tiles. Ignored for T <= 32. No counterpart in the reference. */
    uint64_t work_bytes;
} bn_ternary_args;

/* norm_rotate (kernels/norm_rotate.comp:3-33, model.rs:690-707): the input of the q/k/v projections. For each row,
 * xn = h * (1 / sqrt(sum h^2 / d + 1e-6)) * w and xr = FWHT-512(signs * xn) / sqrt(512) per 512-element block. */
typedef struct bn_norm_args {
    uint32_t T;              /* rows */
    uint32_t d;              /* row width (the model's hidden size): a multiple of 512 */
    const float* h;          /* row t at h + t * h_ts (16-byte aligned, h_ts a multiple of 4) */
    int64_t h_ts;
    const float* w;          /* [d] RMSNorm weight */
    const float* signs;      /* [d] +-1: the first projection's input signs (model.rs:697, Lin.signs) */
    float* xn;               /* rmsnorm(h) * w rows (write_xn), or NULL */
    int64_t xn_ts;
    float* xr;               /* rotated rows: the projections' x */
    int64_t xr_ts;
    /* the LoRA-A rows of norm_rotate (norm_rotate.comp:21, rot.glsl:19-40): u[t][r] = sum_e A[r][e] * xn[t][e]
     * (rmsnorm(h) * w), in extra blocks of the same launch; the u the q/k/v call's LoRA up projection reads */
    const uint16_t* lora_a;  /* [lora_r][d] fp16, 16-byte aligned, d <= 8192; NULL with lora_r == 0 */
    float* lora_u;           /* out: u[t][r] at lora_u + t * lora_us + r */
    int64_t lora_us;
    uint32_t lora_r;
} bn_norm_args;

/* ---- context ---------------------------------------------------------------------------------- */
bn_status bn_ctx_create(int device, bn_ctx** out);
void bn_ctx_destroy(bn_ctx* ctx);
const char* bn_status_str(bn_status s);
/* Text of the last failed check or launch on this context (empty if none). */
const char* bn_ctx_last_error(const bn_ctx* ctx);
int bn_abi_version(void);
/* Reads and clears this context's device's overflow flag: *flag = 1 if any call since the last read found a device
 * offset (dyn[0]) above its host bound `off` (the call then attended as at `off` and appended nothing), else 0.
 * No counterpart in the reference (a Vulkan dispatch past its bound is undefined there). Synchronous: call it
 * after the stream work that read the offsets has finished. Calls on one device share the flag. */
bn_status bn_dyn_overflow(bn_ctx* ctx, int* flag);

/* ---- sizes and checks (pure host code, no device access) ----------------------------------------- */
size_t bn_attn_workspace_size(const bn_attn_args* a);
size_t bn_ragged_workspace_size(const bn_ragged_args* a);
/* kind: 0 forward (any T), 1 decode (T == 1), 2 verify (T <= 16), 3 prefill (any T), 4 append only */
bn_status bn_attn_check(const bn_attn_args* a, int kind);
bn_status bn_ragged_check(const bn_ragged_args* a);

/* Zero-fills device memory on `stream` with a kernel (no memset node: safe inside graph capture). The
 * attention calls do not need it; it is there for callers that keep their own scratch next to the workspace. */
bn_status bn_workspace_clear(bn_ctx* ctx, bn_stream stream, void* ws, size_t bytes);

/* ---- the attention call ------------------------------------------------------------------------- */
/* Appends k_new/v_new, attends, gates. Chooses the decode, verify or prefill kernel from T
 * (model.rs:852-855 chooses the reference's split chunk the same way). */
bn_status bn_attn_forward(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a);
/* The same call with the kernel fixed; T must fit the kernel (decode: T == 1; verify: T <= 16). */
bn_status bn_attn_decode(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a);
bn_status bn_attn_verify(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a);
bn_status bn_attn_prefill(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a);
/* Cache append only: rows [off, off + T) of kc/vc from k_new/v_new (attn_prep.comp:36-39,58, fp16 store). */
bn_status bn_attn_append(bn_ctx* ctx, bn_stream stream, const bn_attn_args* a);

/* Ragged batched decode: no counterpart in the reference (one sequence per model there); each sequence
 * is the decode call above with its own cache rows. */
bn_status bn_attn_decode_ragged(bn_ctx* ctx, bn_stream stream, const bn_ragged_args* a);
/* The same call without a workspace, for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc); no counterpart in the reference. a->ws and
 * a->ws_bytes are ignored: the split partials go to a library-owned array of BN_NOALLOC_SCRATCH_BYTES
 * (16 MiB) that each device holds from the library's load until the process ends. A batch whose partials
 * need more is rejected with BN_ENOWS before any launch (32 sequences x 4 kv heads need 4.8 MB with the
 * default split policy). The call allocates nothing and needs no initialisation of the array. Every call on
 * one device shares that device's array, so calls that overlap in time on one device (on different streams)
 * race. */
bn_status bn_attn_decode_ragged_noalloc(bn_ctx* ctx, bn_stream stream, const bn_ragged_args* a);
#define BN_NOALLOC_SCRATCH_BYTES (16u << 20)

/* ---- prefix-state snapshots -------------------------------------------------------------------------- */
/* encode_copy_state's KV part: rows [0, from->len) of every layer from `from` into `to` (same n_layers and KV,
 * to->cap >= from->len); one kernel on `stream` for both caches (two 2-D device copies when a cache pointer is not
 * 16-byte aligned). The caches must not overlap. to->len is the caller's to set. */
bn_status bn_kv_copy(bn_ctx* ctx, bn_stream stream, const bn_kv_state* from, const bn_kv_state* to);
/* Bytes of s's KV section (header + 2 * n_layers * len * KV * 256 * 2); 0 for a bad state. */
size_t bn_kv_section_size(const bn_kv_state* s);
/* Writes s's KV section (rows [0, s->len)) to host memory `dst` of dst_bytes >= bn_kv_section_size(s); waits for
 * the copies, so `dst` is complete on return. */
bn_status bn_kv_section_save(bn_ctx* ctx, bn_stream stream, const bn_kv_state* s, void* dst, size_t dst_bytes);
/* Checks a KV section against s (magic, version, n_layers, KV, len <= s->cap, size) without device access and
 * gives its len. */
bn_status bn_kv_section_check(const void* src, size_t src_bytes, const bn_kv_state* s, uint32_t* len_out);
/* Loads a checked section into rows [0, len) of s's caches (load_prefix's gpu::write of the KV parts); rows past
 * len are untouched. Waits for the copies. A section that fails the check leaves the device untouched. */
bn_status bn_kv_section_load(bn_ctx* ctx, bn_stream stream, const void* src, size_t src_bytes, const bn_kv_state* s,
                             uint32_t* len_out);

/* ---- either side of the attention call ------------------------------------------------------------ */
bn_status bn_prep_check(const bn_prep_args* a);
bn_status bn_rotate_check(const bn_rotate_args* a);
bn_status bn_layer_check(const bn_prep_args* p, const bn_attn_args* a);
/* attn_prep (kernels/attn_prep.comp:29-59): norms, mRoPE, fp16 K/V append. */
bn_status bn_attn_prep(bn_ctx* ctx, bn_stream stream, const bn_prep_args* a);
/* gate_rotate (kernels/gate_rotate.comp:11-26): gate, signs, FWHT-512, 1/sqrt(512); `xr` is o_proj's input; with
 * lora_r > 0 also the LoRA-A rows u of the gated row. */
bn_status bn_gate_rotate(bn_ctx* ctx, bn_stream stream, const bn_rotate_args* a);

/* The attention arm of one layer in one call (model.rs:828-893: attn_prep, attn_split, attn_combine, gate_rotate):
 * p's raw rows (q_proj's q half, k_proj, v_proj) are normed and rotated as bn_attn_prep does, the K/V rows land
 * in the cache, and `a` attends, gates and (with a->signs) rotates. One row (a decode step) runs attn_prep inside
 * the decode kernel's prologue: one split launch, plus the split merge when the keys are split. 2..16 rows whose
 * keys the workspace splits (verify drafts) have q and the K/V rows written by the prep kernel (q to p->q in p's
 * form when given, else fp32 into the workspace), then the verify kernel and the merge. Other rows up to 16 (short
 * contexts) run as decodes of their rows with q normed in the prologue, their K/V rows written by the prep kernel
 * first. For T > 16 (prefill) the
 * prep kernel writes q to p->q (fp16 with BN_Q_F16, the faster form for the prefill kernels) and the K/V rows,
 * then the prefill kernels run. p and a describe the same rows (T, off, H, KV, cap, kc, vc); a->q, a->k_new and
 * a->v_new are NULL and a->flags is 0. p->q is needed only for T > 16; otherwise it may be NULL (when given for
 * 2..16 rows it receives q). Same workspace as bn_attn_forward. */
bn_status bn_attn_layer(bn_ctx* ctx, bn_stream stream, const bn_prep_args* p, const bn_attn_args* a);

/* ---- ternary projections either side of the attention call ------------------------------------------ */
bn_status bn_norm_check(const bn_norm_args* a);
/* norm_rotate: the q/k/v projections' input from the hidden rows (one launch, one wave per 512-element block), and
 * with lora_r > 0 the LoRA down projection u of the normed rows (rot.glsl LORA_ROW) in extra blocks of the launch. */
bn_status bn_norm_rotate(bn_ctx* ctx, bn_stream stream, const bn_norm_args* a);
bn_status bn_ternary_check(const bn_ternary_args* a);
/* y = (add ? y : 0) + x W^T (+ LoRA) for each matrix (model.rs:455-596: qmm_multi / qmv4 for one token, qmvr,
 * qmvx and qmm3 for more; kernels.metal:431-500 qmm, 664-709 qmvxm). Results are fp32 sums of exact products up to
 * x's 2^-22 relative split error (the reference computes in fp32), identical from call to call, for any finite x
 * up to about 4e9 in magnitude (x beyond fp16's range is scaled by a power of two inside the call). y must not
 * overlap x, W or another matrix's y. */
bn_status bn_ternary_matmul(bn_ctx* ctx, bn_stream stream, const bn_ternary_args* a);
/* Bytes of bn_ternary_args.work for T tokens of width k (0 when T <= 32: those calls use none). With a workspace the
 * call runs two kernels: x split into fp16 pairs once, then the GEMM streaming those tiles (scale arrays that are not
 * 4-byte aligned fall back to the GEMM that splits in place). Results are identical either way. */
size_t bn_ternary_workspace_size(uint32_t T, uint32_t k);

#ifdef __cplusplus
}
#endif
#endif
