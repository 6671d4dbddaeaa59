//! Raw FFI to libllmoxide_amd (HIP, gfx950): the entry points that replace the
//! attention, KV-append and gated-delta-rule dispatches llmoxide's
//! `crates/gpu` records.  A one-to-one mirror of `include/lmx/attn.h`, which is
//! the authority for every type, argument and contract; `tests/test_rust_ffi.py`
//! parses both files and fails when they drift apart.
//!
//! Conventions (the header's): device pointers are caller-owned HIP
//! allocations; no entry point allocates, frees or synchronizes the host; work
//! is enqueued on `stream` (a `hipStream_t`, NULL for the null stream); a
//! rejected call returns an `LMX_E_*` code and enqueues nothing.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_void, CStr};
use std::fmt;

/// `lmx_stream`: binary-compatible with `hipStream_t`.
pub type HipStream = *mut c_void;

/// `lmx_status` codes.
pub const LMX_OK: i32 = 0;
pub const LMX_E_NULL: i32 = 1;
pub const LMX_E_SHAPE: i32 = 2;
pub const LMX_E_UNSUPPORTED: i32 = 3;
pub const LMX_E_WORKSPACE: i32 = 4;
pub const LMX_E_CONTEXT: i32 = 5;
pub const LMX_E_RING_HAZARD: i32 = 6;
pub const LMX_E_ALIGN: i32 = 7;
pub const LMX_E_LAUNCH: i32 = 8;
pub const LMX_E_DEVICE: i32 = 9;
pub const LMX_E_FULL: i32 = 10;
pub const LMX_E_HOST: i32 = 11;

/// `lmx_dtype`.
pub const LMX_F32: i32 = 0;
pub const LMX_F16: i32 = 1;

/// `LMX_NOALLOC_SCRATCH_BYTES`: the per-GPU scratch of `lmx_attn_fwd_noalloc`.
pub const LMX_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

/// `lmx_attn_params`: the `Attn` uniform (attn.wgsl:22-34, qwen35.rs:36-49,
/// forward.rs:29-44) without `max_vis`, plus `n_slots`.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LmxAttnParams {
    pub n_tokens: u32,
    pub n_heads: u32,
    pub n_kv_heads: u32,
    pub head_dim: u32,
    pub kv_dim: u32,
    pub base_pos: u32,
    pub window: u32,
    pub n_slots: u32,
    pub bidi: u32,
    pub scale: f32,
}

/// `lmx_kv_desc`: write_cache's view of one append (ops.wgsl:323-346).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LmxKvDesc {
    pub n_tokens: u32,
    pub kv_dim: u32,
    pub base_pos: u32,
    pub window: u32,
    pub n_slots: u32,
}

/// `lmx_dop`: the `DOp` uniform (deltanet.wgsl:20-34, qwen35.rs:51-68), the
/// fields the recurrence reads.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LmxDop {
    pub n_tok: u32,
    pub conv_dim: u32,
    pub key_dim: u32,
    pub d_inner: u32,
    pub s_dim: u32,
    pub n_vh: u32,
    pub n_kh: u32,
    pub scale: f32,
}

/// `lmx_prologue_desc`: geometry of the norm / rotate / store prologue.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LmxPrologueDesc {
    pub n_tokens: u32,
    pub n_heads: u32,
    pub n_kv_heads: u32,
    pub head_dim: u32,
    pub q_stride: u32,
    pub n_rot: u32,
    pub base_pos: u32,
    pub window: u32,
    pub n_slots: u32,
    pub v_norm: u32,
    pub rms_eps: f32,
    pub rope_base: f32,
}

/// `lmx_attn_ext`: query head stride and optional sigmoid output gate
/// (Qwen3.5's fused `[query | gate]` heads).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct LmxAttnExt {
    pub q_stride: u32,
    pub gate_stride: u32,
    pub gate: *const f32,
}

/// `lmx_delta_front_desc`: conv / window / q-k norm front of the delta-net.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LmxDeltaFrontDesc {
    pub n_tok: u32,
    pub conv_dim: u32,
    pub key_dim: u32,
    pub s_dim: u32,
    pub kernel: u32,
    pub eps: f32,
}

/// `lmx_delta_back_desc`: the gated RMS norm after the recurrence.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LmxDeltaBackDesc {
    pub n_tok: u32,
    pub n_vh: u32,
    pub s_dim: u32,
    pub eps: f32,
}

/// `lmx_qmv_desc`: a GGUF-layout weight matrix (`type` = the ggml type id)
/// times `n_tok` token vectors.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LmxQmvDesc {
    pub r#type: u32,
    pub rows: u32,
    pub in_dim: u32,
    pub n_tok: u32,
}

/// `lmx_kvm_layer`: one layer of a KV manager (window, row size, sharing).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct LmxKvmLayer {
    pub window: u32,
    pub kv_dim: u32,
    pub kv_source: i32,
}

/// `lmx_kvm_desc`: layers, positions per sequence and sequence slots.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct LmxKvmDesc {
    pub n_layers: u32,
    pub n_ctx: u32,
    pub max_seqs: u32,
    pub layers: *const LmxKvmLayer,
}

/// `lmx_kvm`: an opaque KV manager handle.
#[repr(C)]
pub struct LmxKvm {
    _private: [u8; 0],
}

#[link(name = "llmoxide_amd")]
extern "C" {
    pub fn lmx_status_str(s: i32) -> *const c_char;
    pub fn lmx_version() -> i32;
    /// Re-reads the LMX_* kernel-choice overrides (tests and tuning sweeps).
    pub fn lmx_tuning_reload();
    pub fn lmx_workspace_init(ws: *mut c_void, ws_bytes: usize, stream: HipStream) -> i32;

    /// The two `write_cache` dispatches (ops.wgsl:323-346; qwen35.rs:1062-1074,
    /// forward.rs:964-985).
    pub fn lmx_kv_append(d: *const LmxKvDesc, k_new: *const f32, v_new: *const f32, k_cache: *mut c_void,
                         v_cache: *mut c_void, cache_dt: i32, stream: HipStream) -> i32;

    /// rms_norm + rope + rms_norm + rope (+ V norm) + both `write_cache`
    /// dispatches in one launch (qwen35.rs:1030-1074, forward.rs:914-985).
    pub fn lmx_attn_prologue(d: *const LmxPrologueDesc, q: *mut f32, k_new: *const f32, v_new: *const f32,
                             q_gain: *const f32, k_gain: *const f32, rope_factors: *const f32,
                             k_cache: *mut c_void, v_cache: *mut c_void, cache_dt: i32,
                             stream: HipStream) -> i32;

    pub fn lmx_attn_workspace_bytes(p: *const LmxAttnParams) -> usize;

    /// `scores_pass` / `softmax_pass` / `weighted_v` (attn.wgsl:84-232;
    /// qwen35.rs:1076-1094, forward.rs:988-1011).
    pub fn lmx_attn_fwd(p: *const LmxAttnParams, q: *const c_void, q_dt: i32, k_cache: *const c_void,
                        v_cache: *const c_void, kv_dt: i32, k_cur: *const c_void, v_cur: *const c_void,
                        out: *mut f32, ws: *mut c_void, ws_bytes: usize, stream: HipStream) -> i32;

    /// `lmx_attn_fwd` with the partials in a library-owned per-GPU scratch of
    /// LMX_NOALLOC_SCRATCH_BYTES (no reference counterpart: for callers that
    /// cannot allocate).
    pub fn lmx_attn_fwd_noalloc(p: *const LmxAttnParams, q: *const c_void, q_dt: i32, k_cache: *const c_void,
                                v_cache: *const c_void, kv_dt: i32, k_cur: *const c_void,
                                v_cur: *const c_void, out: *mut f32, stream: HipStream) -> i32;

    /// `lmx_attn_fwd` reading Qwen3.5's fused heads in place and applying the
    /// sigmoid gate (qwen35.rs:1012-1028, 1098-1107; ops.wgsl:150-184).
    pub fn lmx_attn_fwd_ext(p: *const LmxAttnParams, x: *const LmxAttnExt, q: *const c_void, q_dt: i32,
                            k_cache: *const c_void, v_cache: *const c_void, kv_dt: i32,
                            k_cur: *const c_void, v_cur: *const c_void, out: *mut f32, ws: *mut c_void,
                            ws_bytes: usize, stream: HipStream) -> i32;

    pub fn lmx_attn_decode_batched_workspace_bytes(p: *const LmxAttnParams, n_seq: i32, max_ctx: i32) -> usize;

    /// One query per sequence over ragged caches (the reference serves one
    /// sequence: docs/limitations.md:21).
    pub fn lmx_attn_decode_batched(p: *const LmxAttnParams, n_seq: i32, max_ctx: i32, ctx_lens: *const i32,
                                   k_ptrs: *const *const c_void, v_ptrs: *const *const c_void,
                                   q: *const c_void, q_dt: i32, kv_dt: i32, out: *mut f32,
                                   ws: *mut c_void, ws_bytes: usize, stream: HipStream) -> i32;

    /// `delta_recur` (deltanet.wgsl:193-239; qwen35.rs:960-965).
    pub fn lmx_deltanet_recur(op: *const LmxDop, ssm_a: *const f32, dt_bias: *const f32, alpha: *const f32,
                              beta: *const f32, conv: *const f32, state: *mut f32, out: *mut f32,
                              stream: HipStream) -> i32;

    pub fn lmx_deltanet_chunked_workspace_bytes(op: *const LmxDop, chunk: i32) -> usize;

    /// The prefill form of `delta_recur`, chunked (same contract).
    pub fn lmx_deltanet_chunked(op: *const LmxDop, ssm_a: *const f32, dt_bias: *const f32,
                                alpha: *const f32, beta: *const f32, conv: *const f32, state: *mut f32,
                                out: *mut f32, chunk: i32, ws: *mut c_void, ws_bytes: usize,
                                stream: HipStream) -> i32;

    /// conv_silu + conv_shift + conv_commit + l2norm_qk (deltanet.wgsl:54-173;
    /// qwen35.rs:928-958).
    pub fn lmx_deltanet_front(d: *const LmxDeltaFrontDesc, x: *const f32, taps: *const f32,
                              conv_state: *mut f32, conv_out: *mut f32, stream: HipStream) -> i32;

    /// rms_norm over the v-heads + mul_silu (qwen35.rs:968-986).
    pub fn lmx_deltanet_back(d: *const LmxDeltaBackDesc, o: *mut f32, z: *const f32, w: *const f32,
                             stream: HipStream) -> i32;

    /// The `matvec_*` / `gemm_*` dispatches of a GGUF projection (quant.wgsl,
    /// gemm.wgsl; CPU semantics crates/gguf/src/quant.rs:187-271).
    pub fn lmx_matvec(d: *const LmxQmvDesc, w: *const c_void, x: *const f32, y: *mut f32,
                      stream: HipStream) -> i32;

    /// `KvCache` (cache.rs:65-154) and the session's prefix reuse
    /// (session.rs:497-513, 546-570) for many sequences in one device arena.
    pub fn lmx_kvm_arena_bytes(d: *const LmxKvmDesc) -> usize;
    pub fn lmx_kvm_create(d: *const LmxKvmDesc, arena: *mut c_void, arena_bytes: usize,
                          out: *mut *mut LmxKvm) -> i32;
    pub fn lmx_kvm_destroy(m: *mut LmxKvm);
    pub fn lmx_kvm_open(m: *mut LmxKvm, seq: *mut i32) -> i32;
    pub fn lmx_kvm_close(m: *mut LmxKvm, seq: i32) -> i32;
    pub fn lmx_kvm_len(m: *const LmxKvm, seq: i32, len: *mut u32) -> i32;
    pub fn lmx_kvm_reusable_prefix(m: *const LmxKvm, seq: i32, tokens: *const i32, n: u32,
                                   reuse: *mut u32) -> i32;
    pub fn lmx_kvm_begin(m: *mut LmxKvm, seq: i32, tokens: *const i32, n: u32, reuse: *mut u32,
                         stream: HipStream) -> i32;
    pub fn lmx_kvm_commit(m: *mut LmxKvm, seq: i32, tokens: *const i32, n: u32) -> i32;
    pub fn lmx_kvm_truncate(m: *mut LmxKvm, seq: i32, pos: u32) -> i32;
    pub fn lmx_kvm_wipe(m: *mut LmxKvm, seq: i32, stream: HipStream) -> i32;
    pub fn lmx_kvm_layer_cache(m: *const LmxKvm, seq: i32, layer: u32, k: *mut *mut c_void,
                               v: *mut *mut c_void, n_slots: *mut u32, window: *mut u32) -> i32;
    pub fn lmx_kvm_batch(m: *const LmxKvm, layer: u32, seqs: *const i32, n: u32, extra: u32,
                         k_ptrs: *mut *const c_void, v_ptrs: *mut *const c_void, ctx_lens: *mut i32,
                         max_ctx: *mut i32) -> i32;
}

/// A rejected call: the status code and the library's description of it.
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct LmxError {
    pub status: i32,
    pub message: String,
}

impl fmt::Display for LmxError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "libllmoxide_amd: {} (status {})", self.message, self.status)
    }
}

impl std::error::Error for LmxError {}

impl LmxError {
    /// Whether the reference would report this as `Error::ContextOverflow`
    /// (llmoxide/src/error.rs:9-47); `LMX_E_DEVICE` maps to `Error::NoDevice`,
    /// everything else to `Error::Other` with `message`.
    pub fn is_context_overflow(&self) -> bool {
        self.status == LMX_E_CONTEXT
    }
    pub fn is_no_device(&self) -> bool {
        self.status == LMX_E_DEVICE
    }
}

/// Turns a status code into a `Result`.
pub fn check(code: i32) -> Result<(), LmxError> {
    if code == LMX_OK {
        return Ok(());
    }
    // SAFETY: lmx_status_str returns a pointer to static storage for any code.
    let message = unsafe { CStr::from_ptr(lmx_status_str(code)) }.to_string_lossy().into_owned();
    Err(LmxError { status: code, message })
}

#[cfg(test)]
mod tests {
    use super::*;
    use std::mem::{align_of, size_of};

    // The C layouts (include/lmx/attn.h) on LP64: u32/f32 fields of 4 bytes,
    // pointers of 8.
    #[test]
    fn struct_layouts_match_the_header() {
        assert_eq!(size_of::<LmxAttnParams>(), 40);
        assert_eq!(size_of::<LmxKvDesc>(), 20);
        assert_eq!(size_of::<LmxDop>(), 32);
        assert_eq!(size_of::<LmxPrologueDesc>(), 48);
        assert_eq!(size_of::<LmxAttnExt>(), 16);
        assert_eq!(align_of::<LmxAttnExt>(), 8);
        assert_eq!(size_of::<LmxDeltaFrontDesc>(), 24);
        assert_eq!(size_of::<LmxDeltaBackDesc>(), 16);
        assert_eq!(size_of::<LmxQmvDesc>(), 16);
        assert_eq!(size_of::<LmxKvmLayer>(), 12);
        assert_eq!(size_of::<LmxKvmDesc>(), 24);
    }
}
