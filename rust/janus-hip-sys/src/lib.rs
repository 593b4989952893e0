//! Raw FFI binding of libjanus_hip (the C ABI of include/janus_hip.h and
//! include/janus_model.h), one item per declaration, in header order. The
//! safe layer (`compute::ops` over these calls) is the reference crate's own
//! operator functions with their bodies replaced; see INTEGRATION.md.
#![allow(non_camel_case_types)]
#![no_std]

pub use core::ffi::{c_char, c_float, c_int, c_void};

/// Opaque context (one HIP stream, workspaces): `janus_create` / `janus_destroy`.
#[repr(C)]
pub struct janus_ctx {
    _p: [u8; 0],
}
/// Opaque device weight handle: `janus_weight_upload` / `janus_weight_free`.
#[repr(C)]
pub struct janus_weight {
    _p: [u8; 0],
}
/// Opaque decode driver: `janus_model_create` / `janus_model_destroy`.
#[repr(C)]
pub struct janus_model {
    _p: [u8; 0],
}
/// Per-token callback of `janus_model_generate_stream` (`None` is NULL):
/// nonzero to go on, 0 to stop with this token kept.
pub type janus_token_callback = Option<unsafe extern "C" fn(user: *mut c_void, token: u32, index: u32) -> c_int>;

// ---- constants (enums and #defines of the headers) ----
pub const JANUS_OK: c_int = 0;
pub const JANUS_E_INVALID_ARG: c_int = 1;
pub const JANUS_E_INVALID_DIM: c_int = 2;
pub const JANUS_E_UNSUPPORTED_DTYPE: c_int = 3;
pub const JANUS_E_KV_OVERFLOW: c_int = 4;
pub const JANUS_E_TOKEN_RANGE: c_int = 5;
pub const JANUS_E_HIP: c_int = 6;
pub const JANUS_E_OOM: c_int = 7;
pub const JANUS_E_NO_DEVICE: c_int = 8;
pub const JANUS_E_NAN_LOGITS: c_int = 9;
pub const JANUS_DT_F32: c_int = 0;
pub const JANUS_DT_F16: c_int = 1;
pub const JANUS_DT_Q4_0: c_int = 2;
pub const JANUS_DT_Q8_0: c_int = 8;
pub const JANUS_DT_Q4_K: c_int = 12;
pub const JANUS_DT_Q5_K: c_int = 13;
pub const JANUS_DT_Q6_K: c_int = 14;
pub const JANUS_ABI_VERSION: c_int = 1;
pub const JANUS_WEIGHT_FTZ_F16: u32 = 1;
pub const JANUS_WEIGHT_Q6K_REF_ORDER: u32 = 2;
pub const JANUS_TIE_LAST: c_int = 0;
pub const JANUS_TIE_WGSL: c_int = 1;
pub const JANUS_ATTN_SCRATCH_BYTES: usize = 0x1000000;
pub const JANUS_SAMPLER_ARGMAX: c_int = 0;
pub const JANUS_SAMPLER_PENALTY: c_int = 1;
pub const JANUS_SAMPLER_WGSL: c_int = 2;

/// Model shape and precision choices (`ModelConfig`, model/transformer/mod.rs:79-110).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct janus_model_config {
    /// embedding_length
    pub hidden: u32,
    /// attention.head_count
    pub heads: u32,
    /// attention.head_count_kv
    pub kv_heads: u32,
    /// hidden / heads (config.rs:437)
    pub head_dim: u32,
    /// feed_forward_length
    pub ffn: u32,
    pub vocab: u32,
    /// block_count
    pub layers: u32,
    /// KV capacity per sequence
    pub max_seq_len: u32,
    /// sequences per decode step (1 .. 64)
    pub max_batch: u32,
    /// attention.layer_norm_rms_epsilon
    pub rms_eps: c_float,
    /// rope.freq_base
    pub rope_theta: c_float,
    /// JANUS_DT_F32 (the reference's cache, core.rs:60-88) or JANUS_DT_F16
    pub kv_dtype: c_int,
    /// activations entering the matrix products: F32 (reference) or F16
    pub act_dtype: c_int,
}

unsafe extern "C" {
    // ---- include/janus_hip.h ----
    pub fn janus_create(hip_device: c_int, out: *mut *mut janus_ctx) -> c_int;
    pub fn janus_destroy(ctx: *mut janus_ctx);
    pub fn janus_last_error(ctx: *const janus_ctx) -> *const c_char;
    pub fn janus_status_string(status: c_int) -> *const c_char;
    pub fn janus_abi_version() -> c_int;
    pub fn janus_set_stream(ctx: *mut janus_ctx, hip_stream: *mut c_void) -> c_int;
    pub fn janus_get_stream(ctx: *mut janus_ctx) -> *mut c_void;
    pub fn janus_sync(ctx: *mut janus_ctx) -> c_int;
    pub fn janus_workspace_bytes(
        ctx: *const janus_ctx,
        attn_bytes: *mut usize,
        gemm_bytes: *mut usize,
    ) -> c_int;
    pub fn janus_device_count(count: *mut c_int) -> c_int;
    pub fn janus_alloc(ctx: *mut janus_ctx, bytes: usize, d_ptr: *mut *mut c_void) -> c_int;
    pub fn janus_free(ctx: *mut janus_ctx, d_ptr: *mut c_void) -> c_int;
    pub fn janus_h2d(ctx: *mut janus_ctx, d_dst: *mut c_void, h_src: *const c_void, bytes: usize) -> c_int;
    pub fn janus_d2h(ctx: *mut janus_ctx, h_dst: *mut c_void, d_src: *const c_void, bytes: usize) -> c_int;
    pub fn janus_weight_upload(
        ctx: *mut janus_ctx,
        ggml_type: c_int,
        n: u32,
        k: u32,
        bytes: *const c_void,
        nbytes: usize,
        flags: u32,
        out: *mut *mut janus_weight,
    ) -> c_int;
    pub fn janus_weight_free(ctx: *mut janus_ctx, w: *mut janus_weight) -> c_int;
    pub fn janus_weight_info(
        w: *const janus_weight,
        ggml_type: *mut c_int,
        n: *mut u32,
        k: *mut u32,
        device_bytes: *mut usize,
    ) -> c_int;
    pub fn janus_weight_dequant(ctx: *mut janus_ctx, w: *const janus_weight, d_out: *mut c_float) -> c_int;
    pub fn janus_gemm_auto(
        ctx: *mut janus_ctx,
        a: *const c_void,
        a_dtype: c_int,
        w: *const janus_weight,
        c: *mut c_void,
        c_dtype: c_int,
        batch: u32,
        m: u32,
        k: u32,
        n: u32,
    ) -> c_int;
    pub fn janus_gemm_residual(
        ctx: *mut janus_ctx,
        a: *const c_void,
        a_dtype: c_int,
        w: *const janus_weight,
        residual: *const c_float,
        c: *mut c_float,
        rows: u32,
        k: u32,
        n: u32,
    ) -> c_int;
    pub fn janus_rmsnorm(
        ctx: *mut janus_ctx,
        in_: *const c_float,
        out: *mut c_void,
        out_dtype: c_int,
        gamma: *const c_float,
        batch: u32,
        hidden: u32,
        eps: c_float,
    ) -> c_int;
    pub fn janus_silu(ctx: *mut janus_ctx, in_: *const c_float, out: *mut c_float, size: u32) -> c_int;
    pub fn janus_elementwise_mul(
        ctx: *mut janus_ctx,
        a: *const c_float,
        b: *const c_float,
        out: *mut c_float,
        size: u32,
    ) -> c_int;
    pub fn janus_add_tensors(
        ctx: *mut janus_ctx,
        a: *const c_float,
        b: *const c_float,
        out: *mut c_float,
        size: u32,
    ) -> c_int;
    pub fn janus_swiglu(
        ctx: *mut janus_ctx,
        gate: *const c_float,
        up: *const c_float,
        out: *mut c_void,
        out_dtype: c_int,
        size: u32,
    ) -> c_int;
    pub fn janus_rope_table(
        ctx: *mut janus_ctx,
        d_table: *mut c_float,
        max_seq: u32,
        head_dim: u32,
        theta_base: c_float,
    ) -> c_int;
    pub fn janus_rope(
        ctx: *mut janus_ctx,
        in_: *const c_float,
        out: *mut c_float,
        d_table: *const c_float,
        batch: u32,
        heads: u32,
        head_dim: u32,
        position: u32,
        d_positions: *const i32,
    ) -> c_int;
    pub fn janus_kv_update(
        ctx: *mut janus_ctx,
        k_new: *const c_float,
        v_new: *const c_float,
        k_cache: *mut c_void,
        v_cache: *mut c_void,
        kv_dtype: c_int,
        batch: u32,
        kv_heads: u32,
        head_dim: u32,
        position: u32,
        max_seq_len: u32,
        d_row_base: *const i32,
        d_positions: *const i32,
    ) -> c_int;
    pub fn janus_attention(
        ctx: *mut janus_ctx,
        q: *const c_float,
        k_cache: *const c_void,
        v_cache: *const c_void,
        kv_dtype: c_int,
        out: *mut c_float,
        batch: u32,
        heads: u32,
        kv_heads: u32,
        head_dim: u32,
        seq_len: u32,
        max_seq_len: u32,
        d_row_base: *const i32,
        d_seq_lens: *const i32,
        max_len_hint: u32,
        scale: c_float,
    ) -> c_int;
    pub fn janus_attention_noalloc(
        ctx: *mut janus_ctx,
        q: *const c_float,
        k_cache: *const c_void,
        v_cache: *const c_void,
        kv_dtype: c_int,
        out: *mut c_float,
        batch: u32,
        heads: u32,
        kv_heads: u32,
        head_dim: u32,
        seq_len: u32,
        max_seq_len: u32,
        d_row_base: *const i32,
        d_seq_lens: *const i32,
        max_len_hint: u32,
        scale: c_float,
    ) -> c_int;
    pub fn janus_embed(
        ctx: *mut janus_ctx,
        table: *const janus_weight,
        h_ids: *const u32,
        batch: u32,
        out: *mut c_float,
    ) -> c_int;
    pub fn janus_embed_device(
        ctx: *mut janus_ctx,
        table: *const janus_weight,
        d_ids: *const i32,
        batch: u32,
        out: *mut c_float,
    ) -> c_int;
    pub fn janus_argmax(
        ctx: *mut janus_ctx,
        logits: *const c_float,
        d_out: *mut i32,
        vocab: u32,
        batch: u32,
        tie_rule: c_int,
    ) -> c_int;
    pub fn janus_repetition_penalty(
        ctx: *mut janus_ctx,
        logits: *mut c_float,
        vocab: u32,
        d_context: *const i32,
        n_context: u32,
        penalty: c_float,
    ) -> c_int;
    // ---- include/janus_model.h ----
    pub fn janus_model_create(
        ctx: *mut janus_ctx,
        cfg: *const janus_model_config,
        out: *mut *mut janus_model,
    ) -> c_int;
    pub fn janus_model_destroy(m: *mut janus_model);
    pub fn janus_model_set_tensor(
        m: *mut janus_model,
        name: *const c_char,
        ggml_type: c_int,
        n: u32,
        k: u32,
        bytes: *const c_void,
        nbytes: usize,
    ) -> c_int;
    pub fn janus_model_validate(m: *mut janus_model) -> c_int;
    pub fn janus_model_reset(m: *mut janus_model) -> c_int;
    pub fn janus_model_set_kv_cache(
        m: *mut janus_model,
        d_k: *mut c_void,
        d_v: *mut c_void,
        bytes_each: usize,
    ) -> c_int;
    pub fn janus_model_forward(
        m: *mut janus_model,
        tokens: *const u32,
        positions: *const u32,
        nseq: u32,
    ) -> c_int;
    pub fn janus_model_forward_slots(
        m: *mut janus_model,
        tokens: *const u32,
        positions: *const u32,
        slots: *const u32,
        nseq: u32,
    ) -> c_int;
    pub fn janus_model_logits(m: *const janus_model) -> *const c_float;
    pub fn janus_model_kv_cache(m: *const janus_model, which: c_int) -> *mut c_void;
    pub fn janus_model_read_logits(m: *mut janus_model, h_out: *mut c_float, nseq: u32) -> c_int;
    pub fn janus_model_generate(
        m: *mut janus_model,
        prompt: *const u32,
        n_prompt: u32,
        max_tokens: u32,
        repetition_penalty: c_float,
        out_tokens: *mut u32,
        n_out: *mut u32,
    ) -> c_int;
    pub fn janus_model_generate_stream(
        m: *mut janus_model,
        prompt: *const u32,
        n_prompt: u32,
        max_tokens: u32,
        repetition_penalty: c_float,
        cb: janus_token_callback,
        user: *mut c_void,
        out_tokens: *mut u32,
        n_out: *mut u32,
    ) -> c_int;
    pub fn janus_model_generate_batch(
        m: *mut janus_model,
        prompts: *const u32,
        prompt_lens: *const u32,
        nreq: u32,
        max_tokens: u32,
        repetition_penalty: c_float,
        out_tokens: *mut u32,
        n_out: *mut u32,
    ) -> c_int;
    pub fn janus_model_set_sampler(m: *mut janus_model, mode: c_int, repetition_penalty: c_float) -> c_int;
    pub fn janus_model_graph_begin(
        m: *mut janus_model,
        tokens: *const u32,
        positions: *const u32,
        nseq: u32,
    ) -> c_int;
    pub fn janus_model_graph_begin_slots(
        m: *mut janus_model,
        tokens: *const u32,
        positions: *const u32,
        slots: *const u32,
        nseq: u32,
    ) -> c_int;
    pub fn janus_model_graph_run(m: *mut janus_model, steps: u32) -> c_int;
    pub fn janus_model_graph_read_tokens(m: *mut janus_model, h_tokens: *mut u32, nseq: u32) -> c_int;
    pub fn janus_model_read_generated(
        m: *mut janus_model,
        row: u32,
        h_tokens: *mut u32,
        cap: u32,
        n: *mut u32,
    ) -> c_int;
}
