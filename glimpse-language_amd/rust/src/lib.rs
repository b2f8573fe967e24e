//! Binding of libbonsai_attn, the gfx950 full-attention path of the Bonsai runtime, for its HIP backend.
//!
//! The raw items below mirror `include/bonsai_attn.h` one for one: the argument structs field by field
//! (`#[repr(C)]`, C names lower-cased, `dyn` spelled `dyn_`), the constants and every function. `Ctx` and
//! `Ctx::check` are the thin safe layer: a non-zero status becomes an `Err` carrying the library's message, where
//! the reference panics on a shape assert (model.rs:671-672) or a GPU error (gpu_vk.rs:1144) and handle.rs:221-230
//! turns the panic into `BonsaiErrorKind::Runtime`. Device memory, streams and graphs stay the caller's (hipMalloc,
//! hipStream_t through `bn_stream`), as in the C ABI.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void, CStr};

pub const BN_HEAD_DIM: u32 = 256;
pub const BN_ABI_VERSION: c_int = 6;
pub const BN_Q_F16: u32 = 1;
pub const BN_NOALLOC_SCRATCH_BYTES: u32 = 16 << 20;
pub const BN_KV_SECTION_MAGIC: &[u8; 8] = b"BNKVF16\0";
pub const BN_KV_SECTION_VERSION: u32 = 1;
pub const BN_KV_SECTION_HEADER: usize = 24;

pub type bn_status = c_int;
pub const BN_OK: bn_status = 0;
pub const BN_EINVAL: bn_status = 1;
pub const BN_ENOWS: bn_status = 2;
pub const BN_ELAUNCH: bn_status = 3;
pub const BN_EDEVICE: bn_status = 4;

/// bn_attn_check's `kind`
pub const BN_KIND_FORWARD: c_int = 0;
pub const BN_KIND_DECODE: c_int = 1;
pub const BN_KIND_VERIFY: c_int = 2;
pub const BN_KIND_PREFILL: c_int = 3;
pub const BN_KIND_APPEND: c_int = 4;

#[repr(C)]
pub struct bn_ctx {
    _private: [u8; 0],
}

/// a hipStream_t (null: the default stream)
pub type bn_stream = *mut c_void;

/// One attention layer call for T query rows of one sequence.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct bn_attn_args {
    pub t: u32,
    pub off: u32,
    pub h: u32,
    pub kv: u32,
    pub cap: u32,
    pub flags: u32,
    pub q: *const c_void,
    pub q_ts: i64,
    pub q_hs: i64,
    pub k_new: *const f32,
    pub v_new: *const f32,
    pub kc: *mut u16,
    pub vc: *mut u16,
    pub gate: *const f32,
    pub g_ts: i64,
    pub g_hs: i64,
    pub out: *mut f32,
    pub o_ts: i64,
    pub o_hs: i64,
    pub ws: *mut c_void,
    pub ws_bytes: usize,
    pub signs: *const f32,
    pub dyn_: *const u32,
    pub lora_a: *const u16,
    pub lora_u: *mut f32,
    pub lora_us: i64,
    pub lora_r: u32,
}

/// A batch of single-token decodes over sequences of different lengths.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct bn_ragged_args {
    pub nseq: u32,
    pub h: u32,
    pub kv: u32,
    pub max_len: u32,
    pub q: *const f32,
    pub q_ss: i64,
    pub q_hs: i64,
    pub k_new: *const f32,
    pub v_new: *const f32,
    pub kc: *mut u16,
    pub vc: *mut u16,
    pub kv_off: *const i64,
    pub kv_len: *const i32,
    pub gate: *const f32,
    pub g_ss: i64,
    pub g_hs: i64,
    pub out: *mut f32,
    pub o_ss: i64,
    pub o_hs: i64,
    pub ws: *mut c_void,
    pub ws_bytes: usize,
    pub signs: *const f32,
}

/// attn_prep's arguments (q/k RMS-norm, interleaved mRoPE, fp16 K/V append).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct bn_prep_args {
    pub t: u32,
    pub off: u32,
    pub h: u32,
    pub kv: u32,
    pub cap: u32,
    pub flags: u32,
    pub rot: u32,
    pub s1: u32,
    pub s2: u32,
    pub qp: *const f32,
    pub qp_ts: i64,
    pub qp_hs: i64,
    pub kp: *const f32,
    pub vp: *const f32,
    pub q_norm: *const f32,
    pub k_norm: *const f32,
    pub pos: *const i32,
    pub inv_freq: *const f32,
    pub q: *mut c_void,
    pub q_ts: i64,
    pub q_hs: i64,
    pub kc: *mut u16,
    pub vc: *mut u16,
    pub dyn_: *const u32,
}

/// gate_rotate's arguments (gate, signs, FWHT-512, LoRA-A rows).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct bn_rotate_args {
    pub t: u32,
    pub h: u32,
    pub attn: *const f32,
    pub a_ts: i64,
    pub gate: *const f32,
    pub g_ts: i64,
    pub g_hs: i64,
    pub signs: *const f32,
    pub xr: *mut f32,
    pub x_ts: i64,
    pub lora_a: *const u16,
    pub lora_u: *mut f32,
    pub lora_us: i64,
    pub lora_r: u32,
}

/// The attention layers' fp16 caches of a prefix-state snapshot.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct bn_kv_state {
    pub kc: *mut u16,
    pub vc: *mut u16,
    pub n_layers: u32,
    pub kv: u32,
    pub cap: u32,
    pub len: u32,
}

/// One ternary packed linear (Lin: codes, fp16 scales) and its output rows.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct bn_ternary_mat {
    pub w: *const u32,
    pub s: *const u16,
    pub y: *mut f32,
    pub lora_b: *const u16,
    pub o: u32,
    pub y_ts: i64,
}

/// Up to three ternary matmuls sharing one input (q/k/v; o_proj alone with add = 1).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct bn_ternary_args {
    pub t: u32,
    pub k: u32,
    pub x: *const f32,
    pub x_ts: i64,
    pub n_mats: u32,
    pub add: u32,
    pub mat: [bn_ternary_mat; 3],
    pub lora_u: *const f32,
    pub lora_us: i64,
    pub lora_r: u32,
    pub work: *mut c_void,
    pub work_bytes: u64,
}

/// norm_rotate's arguments (the q/k/v projections' input from the hidden rows).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct bn_norm_args {
    pub t: u32,
    pub d: u32,
    pub h: *const f32,
    pub h_ts: i64,
    pub w: *const f32,
    pub signs: *const f32,
    pub xn: *mut f32,
    pub xn_ts: i64,
    pub xr: *mut f32,
    pub xr_ts: i64,
    pub lora_a: *const u16,
    pub lora_u: *mut f32,
    pub lora_us: i64,
    pub lora_r: u32,
}

macro_rules! zeroed_default {
    ($($t:ty),*) => {$(
        impl Default for $t {
            /// every count 0 and every pointer null (the C `{0}`)
            fn default() -> Self {
                // SAFETY: plain integers and raw pointers, for which all-zero bits are valid
                unsafe { std::mem::zeroed() }
            }
        }
    )*};
}
zeroed_default!(bn_attn_args, bn_ragged_args, bn_prep_args, bn_rotate_args, bn_kv_state, bn_ternary_mat,
                bn_ternary_args, bn_norm_args);

extern "C" {
    pub fn bn_ctx_create(device: c_int, out: *mut *mut bn_ctx) -> bn_status;
    pub fn bn_ctx_destroy(ctx: *mut bn_ctx);
    pub fn bn_status_str(s: bn_status) -> *const c_char;
    pub fn bn_ctx_last_error(ctx: *const bn_ctx) -> *const c_char;
    pub fn bn_abi_version() -> c_int;
    pub fn bn_dyn_overflow(ctx: *mut bn_ctx, flag: *mut c_int) -> bn_status;

    pub fn bn_attn_workspace_size(a: *const bn_attn_args) -> usize;
    pub fn bn_ragged_workspace_size(a: *const bn_ragged_args) -> usize;
    pub fn bn_attn_check(a: *const bn_attn_args, kind: c_int) -> bn_status;
    pub fn bn_ragged_check(a: *const bn_ragged_args) -> bn_status;
    pub fn bn_workspace_clear(ctx: *mut bn_ctx, stream: bn_stream, ws: *mut c_void, bytes: usize) -> bn_status;

    pub fn bn_attn_forward(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_attn_args) -> bn_status;
    pub fn bn_attn_decode(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_attn_args) -> bn_status;
    pub fn bn_attn_verify(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_attn_args) -> bn_status;
    pub fn bn_attn_prefill(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_attn_args) -> bn_status;
    pub fn bn_attn_append(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_attn_args) -> bn_status;
    pub fn bn_attn_decode_ragged(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_ragged_args) -> bn_status;
    pub fn bn_attn_decode_ragged_noalloc(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_ragged_args) -> bn_status;

    pub fn bn_kv_copy(ctx: *mut bn_ctx, stream: bn_stream, from: *const bn_kv_state, to: *const bn_kv_state)
        -> bn_status;
    pub fn bn_kv_section_size(s: *const bn_kv_state) -> usize;
    pub fn bn_kv_section_save(ctx: *mut bn_ctx, stream: bn_stream, s: *const bn_kv_state, dst: *mut c_void,
                              dst_bytes: usize) -> bn_status;
    pub fn bn_kv_section_check(src: *const c_void, src_bytes: usize, s: *const bn_kv_state, len_out: *mut u32)
        -> bn_status;
    pub fn bn_kv_section_load(ctx: *mut bn_ctx, stream: bn_stream, src: *const c_void, src_bytes: usize,
                              s: *const bn_kv_state, len_out: *mut u32) -> bn_status;

    pub fn bn_prep_check(a: *const bn_prep_args) -> bn_status;
    pub fn bn_rotate_check(a: *const bn_rotate_args) -> bn_status;
    pub fn bn_layer_check(p: *const bn_prep_args, a: *const bn_attn_args) -> bn_status;
    pub fn bn_attn_prep(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_prep_args) -> bn_status;
    pub fn bn_gate_rotate(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_rotate_args) -> bn_status;
    pub fn bn_attn_layer(ctx: *mut bn_ctx, stream: bn_stream, p: *const bn_prep_args, a: *const bn_attn_args)
        -> bn_status;

    pub fn bn_norm_check(a: *const bn_norm_args) -> bn_status;
    pub fn bn_norm_rotate(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_norm_args) -> bn_status;
    pub fn bn_ternary_check(a: *const bn_ternary_args) -> bn_status;
    pub fn bn_ternary_matmul(ctx: *mut bn_ctx, stream: bn_stream, a: *const bn_ternary_args) -> bn_status;
    pub fn bn_ternary_workspace_size(t: u32, k: u32) -> usize;
}

/// A failed call: its status and the library's message for it.
#[derive(Debug, Clone)]
pub struct Error {
    pub status: bn_status,
    pub message: String,
}

impl std::fmt::Display for Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        // SAFETY: bn_status_str returns a static NUL-terminated string for every value
        let name = unsafe { CStr::from_ptr(bn_status_str(self.status)) }.to_string_lossy();
        write!(f, "bonsai_attn: {}: {}", name, self.message)
    }
}

impl std::error::Error for Error {}

fn message(ctx: *const bn_ctx) -> String {
    // SAFETY: bn_ctx_last_error returns a NUL-terminated string owned by the context (or the library's
    // thread-local check buffer for a null context)
    unsafe { CStr::from_ptr(bn_ctx_last_error(ctx)) }.to_string_lossy().into_owned()
}

/// The status of one of the pure checks (bn_*_check) as a Result.
pub fn check_args(status: bn_status) -> Result<(), Error> {
    if status == BN_OK {
        Ok(())
    } else {
        Err(Error { status, message: message(std::ptr::null()) })
    }
}

/// A library context on one device (bn_ctx_create / bn_ctx_destroy). The C ABI asks callers to serialise calls on
/// one context, as the runtime does behind its model mutex (handle.rs:96-103): `Ctx` is `Send`, not `Sync`.
pub struct Ctx {
    raw: *mut bn_ctx,
}

unsafe impl Send for Ctx {}

impl Ctx {
    pub fn new(device: i32) -> Result<Ctx, Error> {
        // SAFETY: ABI version query and context creation take no pointers but `raw`'s address
        let version = unsafe { bn_abi_version() };
        if version != BN_ABI_VERSION {
            return Err(Error {
                status: BN_EDEVICE,
                message: format!("library ABI version {} where this binding has {}", version, BN_ABI_VERSION),
            });
        }
        let mut raw = std::ptr::null_mut();
        let status = unsafe { bn_ctx_create(device, &mut raw) };
        if status != BN_OK || raw.is_null() {
            return Err(Error { status, message: message(std::ptr::null()) });
        }
        Ok(Ctx { raw })
    }

    pub fn raw(&self) -> *mut bn_ctx {
        self.raw
    }

    /// A call's status as a Result with the context's message for it.
    pub fn check(&self, status: bn_status) -> Result<(), Error> {
        if status == BN_OK {
            Ok(())
        } else {
            Err(Error { status, message: message(self.raw) })
        }
    }

    /// bn_attn_layer: the attention arm of one layer (attn_prep, attn_split, attn_combine, gate_rotate) in one
    /// call on `stream`. The pointers inside `p` and `a` are device memory the caller keeps alive until the
    /// stream has run the call.
    pub unsafe fn attn_layer(&self, stream: bn_stream, p: &bn_prep_args, a: &bn_attn_args) -> Result<(), Error> {
        self.check(bn_attn_layer(self.raw, stream, p, a))
    }

    /// bn_attn_forward: append, attend and gate T rows (the kernel chosen from T).
    pub unsafe fn attn_forward(&self, stream: bn_stream, a: &bn_attn_args) -> Result<(), Error> {
        self.check(bn_attn_forward(self.raw, stream, a))
    }

    /// bn_ternary_matmul: up to three projections sharing one input.
    pub unsafe fn ternary_matmul(&self, stream: bn_stream, a: &bn_ternary_args) -> Result<(), Error> {
        self.check(bn_ternary_matmul(self.raw, stream, a))
    }

    /// bn_norm_rotate: the q/k/v projections' input from the hidden rows.
    pub unsafe fn norm_rotate(&self, stream: bn_stream, a: &bn_norm_args) -> Result<(), Error> {
        self.check(bn_norm_rotate(self.raw, stream, a))
    }
}

impl Drop for Ctx {
    fn drop(&mut self) {
        // SAFETY: raw came from bn_ctx_create and is destroyed once
        unsafe { bn_ctx_destroy(self.raw) }
    }
}
