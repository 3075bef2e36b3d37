//! Raw declarations of `librailgun_hip.so`, the C ABI of `include/railgun_hip.h`.
//!
//! One `extern "C"` declaration per entry of the header, in the header's order, with the
//! same parameter names; `tests/test_rust_crate.py` checks names, parameter counts and
//! types against the header.  Pointers are raw device pointers; every call is `unsafe`
//! because the library trusts its indices, as the CUDA launchers it replaces do.

use std::os::raw::{c_char, c_int, c_void};

pub const RG_ABI_VERSION: c_int = 1;

pub const RG_OK: c_int = 0;
pub const RG_ERR_INVALID_ARGUMENT: c_int = 1;
pub const RG_ERR_NOT_SUPPORTED: c_int = 2;
pub const RG_ERR_HIP: c_int = 3;
pub const RG_ERR_WORKSPACE: c_int = 4;

pub const RG_DTYPE_F32: i32 = 0;
pub const RG_DTYPE_BF16: i32 = 1;
pub const RG_DTYPE_F16: i32 = 2;

pub const RG_MAX_HEAD_DIM: i32 = 256;
pub const RG_NO_ALLOC_SCRATCH_BYTES: usize = 16 << 20;

#[link(name = "railgun_hip")]
extern "C" {
    /// Thread-local message of the last failing call.
    pub fn rg_last_error() -> *const c_char;
    /// RG_ABI_VERSION of the loaded library.
    pub fn rg_abi_version() -> c_int;
    /// Replaces PagedAttentionKernels::new (crates/vllm-cuda/src/kernels/mod.rs:57-190).
    pub fn rg_init(device_ordinal: c_int) -> c_int;
    /// Replaces launch_rope (mod.rs:196-225).
    pub fn rg_rope(
        x: *mut c_void, cos_sin: *const f32, positions: *const i32, num_heads: i32, head_dim: i32,
        num_tokens: i32, dtype: i32, stream: *mut c_void,
    ) -> c_int;
    /// Host helper: the cos/sin table apply_rope takes as input (paged_attn_op.rs:236-268).
    pub fn rg_rope_cos_sin_table(table: *mut f32, max_position: i32, head_dim: i32, theta: f64) -> c_int;
    /// Replaces launch_reshape_and_cache (mod.rs:227-262).
    pub fn rg_reshape_and_cache(
        k: *const c_void, v: *const c_void, k_cache: *mut c_void, v_cache: *mut c_void,
        slot_mapping: *const i32, num_kv_heads: i32, head_dim: i32, block_size: i32, num_tokens: i32,
        dtype: i32, kv_block_stride: i64, stream: *mut c_void,
    ) -> c_int;
    /// Replaces launch_reshape_and_cache_isoquant (mod.rs:264-303).
    pub fn rg_reshape_and_cache_isoquant(
        k: *const c_void, v: *const c_void, k_cache: *mut c_void, v_cache: *mut c_void,
        slot_mapping: *const i32, rotation_metadata: *mut f32, num_kv_heads: i32, head_dim: i32,
        block_size: i32, num_tokens: i32, dtype: i32, kv_block_stride: i64, stream: *mut c_void,
    ) -> c_int;
    /// New: RoPE on q/k and the cache write in one pass.
    pub fn rg_rope_reshape_and_cache(
        q: *mut c_void, k: *const c_void, v: *const c_void, k_cache: *mut c_void, v_cache: *mut c_void,
        cos_sin: *const f32, positions: *const i32, slot_mapping: *const i32, num_heads: i32,
        num_kv_heads: i32, head_dim: i32, block_size: i32, num_tokens: i32, dtype: i32, kv_block_stride: i64,
        stream: *mut c_void,
    ) -> c_int;
    /// New: the same from one fused q/k/v projection output (attention.rs:104-125).
    pub fn rg_qkv_rope_reshape_and_cache(
        qkv: *const c_void, qkv_token_stride: i64, q_out: *mut c_void, k_cache: *mut c_void,
        v_cache: *mut c_void, cos_sin: *const f32, positions: *const i32, slot_mapping: *const i32,
        num_heads: i32, num_kv_heads: i32, head_dim: i32, block_size: i32, num_tokens: i32, dtype: i32,
        kv_block_stride: i64, stream: *mut c_void,
    ) -> c_int;
    /// New: the fused q/k/v projection and rg_qkv_rope_reshape_and_cache in one pass (decode batches).
    pub fn rg_linear_qkv_rope_reshape_and_cache(
        x: *const c_void, weight_qkv: *const c_void, q_out: *mut c_void, k_cache: *mut c_void,
        v_cache: *mut c_void, cos_sin: *const f32, positions: *const i32, slot_mapping: *const i32,
        num_tokens: i32, num_heads: i32, num_kv_heads: i32, head_dim: i32, block_size: i32, in_features: i32,
        x_row_stride: i64, weight_row_stride: i64, q_out_token_stride: i64, kv_block_stride: i64, dtype: i32,
        stream: *mut c_void,
    ) -> c_int;
    /// New: the physical copies behind swap_out / swap_in / fork (allocator.rs:102-153).
    pub fn rg_copy_blocks(
        src_pool: *const c_void, dst_pool: *mut c_void, block_mapping: *const i32, num_pairs: i32,
        block_bytes: i64, src_block_stride_bytes: i64, dst_block_stride_bytes: i64, num_layers: i32,
        src_layer_stride_bytes: i64, dst_layer_stride_bytes: i64, stream: *mut c_void,
    ) -> c_int;
    /// Residual add + RMSNorm around each sublayer (architecture.rs:38-59).
    pub fn rg_rms_norm(
        x: *const c_void, residual: *mut c_void, weight: *const c_void, out: *mut c_void, eps: f32,
        num_rows: i32, hidden_size: i32, dtype: i32, stream: *mut c_void,
    ) -> c_int;
    /// SwiGLU gate of LlamaMLP (architecture.rs:80-84).
    pub fn rg_silu_and_mul(
        gate_up: *const c_void, out: *mut c_void, num_rows: i32, intermediate_size: i32, dtype: i32,
        stream: *mut c_void,
    ) -> c_int;
    /// Workspace size of the split-K form of v1 / v1_plus.
    pub fn rg_paged_attention_v1_workspace_bytes(
        batch_size: i32, num_heads: i32, num_kv_heads: i32, head_dim: i32, block_size: i32,
        max_blocks_per_seq: i32,
    ) -> usize;
    /// New: the decode-step projection x . weight^T (candle's Linear, architecture.rs:38-59, 80-84).
    pub fn rg_linear(
        x: *const c_void, weight: *const c_void, out: *mut c_void, num_rows: i32, out_features: i32,
        in_features: i32, x_row_stride: i64, weight_row_stride: i64, out_row_stride: i64,
        workspace: *mut c_void, workspace_bytes: usize, dtype: i32, stream: *mut c_void,
    ) -> c_int;
    /// Split-K workspace of rg_linear for this shape (0: runs unsplit).
    pub fn rg_linear_workspace_bytes(num_rows: i32, out_features: i32, in_features: i32) -> usize;
    /// New: residual += x . weight^T (the o_proj / down_proj output and the residual add).
    pub fn rg_linear_residual(
        x: *const c_void, weight: *const c_void, residual: *mut c_void, num_rows: i32, out_features: i32,
        in_features: i32, x_row_stride: i64, weight_row_stride: i64, residual_row_stride: i64,
        workspace: *mut c_void, workspace_bytes: usize, dtype: i32, stream: *mut c_void,
    ) -> c_int;
    /// New: RmsNorm folded into the gate/up projection with SiLU·mul.
    pub fn rg_rms_norm_linear_silu_mul(
        x: *const c_void, norm_weight: *const c_void, eps: f32, weight_gate_up: *const c_void, out: *mut c_void,
        num_rows: i32, intermediate_size: i32, in_features: i32, x_row_stride: i64, weight_row_stride: i64,
        out_row_stride: i64, dtype: i32, stream: *mut c_void,
    ) -> c_int;
    /// New: RmsNorm folded into the q/k/v projection with RoPE and the cache write.
    pub fn rg_rms_norm_linear_qkv_rope_reshape_and_cache(
        x: *const c_void, norm_weight: *const c_void, eps: f32, weight_qkv: *const c_void, q_out: *mut c_void,
        k_cache: *mut c_void, v_cache: *mut c_void, cos_sin: *const f32, positions: *const i32,
        slot_mapping: *const i32, num_tokens: i32, num_heads: i32, num_kv_heads: i32, head_dim: i32,
        block_size: i32, in_features: i32, x_row_stride: i64, weight_row_stride: i64, q_out_token_stride: i64,
        kv_block_stride: i64, dtype: i32, stream: *mut c_void,
    ) -> c_int;
    /// New: the gate/up projection and SiLU·mul in one pass (interleaved gate/up weight).
    pub fn rg_linear_silu_mul(
        x: *const c_void, weight_gate_up: *const c_void, out: *mut c_void, num_rows: i32, intermediate_size: i32,
        in_features: i32, x_row_stride: i64, weight_row_stride: i64, out_row_stride: i64, dtype: i32,
        stream: *mut c_void,
    ) -> c_int;
    /// New: opt-in check of the block tables and context lengths (synchronises the stream).
    pub fn rg_validate_block_tables(
        block_table: *const i32, context_lens: *const i32, batch_size: i32, max_blocks_per_seq: i32,
        block_size: i32, num_blocks: i32, stream: *mut c_void,
    ) -> c_int;
    /// New: opt-in check of a slot mapping (synchronises the stream).
    pub fn rg_validate_slot_mapping(slot_mapping: *const i32, num_tokens: i32, num_slots: i64, stream: *mut c_void)
        -> c_int;
    /// Replaces launch_v1 (mod.rs:305-348).
    pub fn rg_paged_attention_v1(
        query: *const c_void, key_cache: *const c_void, value_cache: *const c_void, block_table: *const i32,
        context_lens: *const i32, output: *mut c_void, scale: f32, num_heads: i32, num_kv_heads: i32,
        head_dim: i32, block_size: i32, max_blocks_per_seq: i32, batch_size: i32, dtype: i32,
        kv_block_stride: i64, workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void,
    ) -> c_int;
    /// Replaces launch_v1_plus (mod.rs:350-399).
    pub fn rg_paged_attention_v1_plus(
        query: *const c_void, key_cache: *const c_void, value_cache: *const c_void, block_table: *const i32,
        context_lens: *const i32, output: *mut c_void, rotation_metadata: *const f32, scale: f32,
        num_heads: i32, num_kv_heads: i32, head_dim: i32, block_size: i32, max_blocks_per_seq: i32,
        batch_size: i32, dtype: i32, kv_block_stride: i64, workspace: *mut c_void, workspace_bytes: usize,
        stream: *mut c_void,
    ) -> c_int;
    /// New: RoPE + reshape_and_cache of one new token per sequence fused into v1's launches
    /// (mod.rs:196-225, 227-262, 305-348 as one call); query is read, not rotated in place.
    pub fn rg_rope_reshape_and_cache_paged_attention_v1(
        query: *const c_void, key: *const c_void, value: *const c_void, key_cache: *mut c_void,
        value_cache: *mut c_void, cos_sin: *const f32, positions: *const i32, slot_mapping: *const i32,
        block_table: *const i32, context_lens: *const i32, output: *mut c_void, scale: f32, num_heads: i32,
        num_kv_heads: i32, head_dim: i32, block_size: i32, max_blocks_per_seq: i32, batch_size: i32, dtype: i32,
        kv_block_stride: i64, workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void,
    ) -> c_int;
    /// New, no counterpart: v1 on the library's static scratch, for callers that cannot allocate.
    pub fn rg_paged_attention_v1_no_alloc(
        query: *const c_void, key_cache: *const c_void, value_cache: *const c_void, block_table: *const i32,
        context_lens: *const i32, output: *mut c_void, scale: f32, num_heads: i32, num_kv_heads: i32,
        head_dim: i32, block_size: i32, max_blocks_per_seq: i32, batch_size: i32, dtype: i32,
        kv_block_stride: i64, stream: *mut c_void,
    ) -> c_int;
    /// Scratch size of v2 (tmp_out, exp_sums, max_logits).
    pub fn rg_v2_workspace_bytes(
        batch_size: i32, num_heads: i32, num_partitions: i32, head_dim: i32,
    ) -> usize;
    /// Replaces launch_v2_partition (mod.rs:401-456).
    pub fn rg_paged_attention_v2_partition(
        query: *const c_void, key_cache: *const c_void, value_cache: *const c_void, block_table: *const i32,
        context_lens: *const i32, tmp_out: *mut f32, exp_sums: *mut f32, max_logits: *mut f32,
        rotation_metadata: *const f32, scale: f32, num_heads: i32, num_kv_heads: i32, head_dim: i32,
        block_size: i32, max_blocks_per_seq: i32, num_partitions: i32, batch_size: i32, partition_size: i32,
        dtype: i32, kv_block_stride: i64, stream: *mut c_void,
    ) -> c_int;
    /// Replaces launch_v2_reduce (mod.rs:458-508).
    pub fn rg_paged_attention_v2_reduce(
        output: *mut c_void, exp_sums: *const f32, max_logits: *const f32, tmp_out: *const f32,
        context_lens: *const i32, rotation_metadata: *const f32, num_heads: i32, head_dim: i32,
        num_partitions: i32, batch_size: i32, partition_size: i32, dtype: i32, stream: *mut c_void,
    ) -> c_int;
    /// The v2 branch of PagedAttentionOp::execute in one call (paged_attn_op.rs:108-158).
    pub fn rg_paged_attention_v2(
        query: *const c_void, key_cache: *const c_void, value_cache: *const c_void, block_table: *const i32,
        context_lens: *const i32, output: *mut c_void, scale: f32, num_heads: i32, num_kv_heads: i32,
        head_dim: i32, block_size: i32, max_blocks_per_seq: i32, batch_size: i32, max_context_len: i32,
        partition_size: i32, dtype: i32, kv_block_stride: i64, workspace: *mut c_void,
        workspace_bytes: usize, stream: *mut c_void,
    ) -> c_int;
    /// New: packed causal prefill over the paged cache (attention.rs:128-132 has none).
    pub fn rg_prefill_packed(
        query: *const c_void, key_cache: *const c_void, value_cache: *const c_void, block_table: *const i32,
        context_lens: *const i32, cu_seqlens: *const i32, output: *mut c_void, scale: f32, num_heads: i32,
        num_kv_heads: i32, head_dim: i32, block_size: i32, max_blocks_per_seq: i32, num_seqs: i32,
        num_tokens: i32, max_query_len: i32, dtype: i32, kv_block_stride: i64, stream: *mut c_void,
    ) -> c_int;
}
