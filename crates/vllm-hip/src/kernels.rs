//! `PagedAttentionKernels` on HIP: the launchers of crates/vllm-cuda/src/kernels/mod.rs:23-509,
//! same method names, argument order and meaning, over librailgun_hip instead of PTX modules.
//!
//! Differences a caller sees:
//! * buffers are `HipSlice<T>` (cudarc's `CudaSlice<T>` on CUDA) and `T` is any `KvElement`
//!   (f32 as in the reference, bf16, f16);
//! * the launches go to the stream given to `new` (the candle device's stream on CUDA);
//! * `kv_block_stride` (elements between consecutive cache blocks, 0 = dense
//!   `[NB, H_kv, bs, D]`) lets the launchers address Railgun's fused pool
//!   `[NB, 2, H_kv, bs, D]` (crates/vllm-paged-attention/src/block.rs:70,89-95);
//! * the v2 launchers take the reference's fixed partition size of 256 tokens
//!   (paged_attention_utils.cuh:10);
//! * extra launchers for the entries the reference lacks (split-K v1 with a workspace, the
//!   combined v2, fused RoPE + cache write, packed prefill, block copies, RMSNorm, SwiGLU).
//!
//! Errors map onto `CoreError` as the reference's do (mod.rs:42-54,222,477-482):
//! `RG_ERR_NOT_SUPPORTED` -> `NotSupported { feature: "PagedAttention", .. }`, any other
//! failure -> `Tensor(message)`.

use std::os::raw::{c_int, c_void};
use std::sync::{Arc, Mutex};

use vllm_core::{CoreError, Device, Result as CoreResult};

use crate::buffer::{HipSlice, KvElement};
use crate::ffi;

/// Tokens per partition of the v2 launchers (the reference's PARTITION_SIZE).
pub const V2_PARTITION_SIZE: i32 = 256;

/// The library's message for the last failing call on this thread.
pub fn last_error() -> String {
    // SAFETY: rg_last_error returns a NUL-terminated thread-local string.
    unsafe { std::ffi::CStr::from_ptr(ffi::rg_last_error()) }.to_string_lossy().into_owned()
}

/// Maps an `RG_*` status onto the reference's error variants.
pub fn status(code: c_int) -> CoreResult<()> {
    match code {
        ffi::RG_OK => Ok(()),
        ffi::RG_ERR_NOT_SUPPORTED => Err(CoreError::NotSupported { feature: "PagedAttention", reason: last_error() }),
        _ => Err(CoreError::Tensor(last_error())),
    }
}

/// Launchers of the attention hot path on one HIP device and stream.
#[derive(Debug, Clone)]
pub struct PagedAttentionKernels {
    ordinal: usize,
    stream: *mut c_void,
    kv_block_stride: i64,
    /// Grow-only device workspace of `PagedAttentionOp::execute`'s split-K forms, shared by
    /// the clones of this object (one `Arc<PagedAttentionKernels>` serves every layer,
    /// model.rs:127, while the op itself is built anew for each call, attention.rs:109-116).
    workspace: Arc<Mutex<Option<HipSlice<u8>>>>,
}

// SAFETY: the stream handle may be used from any thread (HIP orders work per stream).
unsafe impl Send for PagedAttentionKernels {}
unsafe impl Sync for PagedAttentionKernels {}

impl PagedAttentionKernels {
    /// PagedAttentionKernels::new (mod.rs:57-190): checks that `ordinal` is a gfx950 device
    /// whose kernels load; nothing is compiled or cached (the code objects are linked in).
    pub fn new(ordinal: usize, stream: *mut c_void) -> CoreResult<Self> {
        // SAFETY: plain calls.
        let abi = unsafe { ffi::rg_abi_version() };
        if abi != ffi::RG_ABI_VERSION {
            return Err(CoreError::DeviceInit {
                device: Device::Cuda(ordinal as u32),
                reason: format!("librailgun_hip ABI version {abi}, this crate expects {}", ffi::RG_ABI_VERSION),
            });
        }
        match unsafe { ffi::rg_init(ordinal as c_int) } {
            ffi::RG_OK => Ok(Self { ordinal, stream, kv_block_stride: 0, workspace: Arc::new(Mutex::new(None)) }),
            _ => Err(CoreError::DeviceInit { device: Device::Cuda(ordinal as u32), reason: last_error() }),
        }
    }

    /// The same launchers for caches whose blocks are `stride` elements apart (Railgun's
    /// fused pool: `2 * num_kv_heads * block_size * head_dim`).
    pub fn with_kv_block_stride(mut self, stride: i64) -> Self {
        self.kv_block_stride = stride;
        self
    }

    pub fn ordinal(&self) -> usize {
        self.ordinal
    }

    pub fn stream(&self) -> *mut c_void {
        self.stream
    }

    pub fn kv_block_stride(&self) -> i64 {
        self.kv_block_stride
    }

    /// Runs `f` with a device workspace of at least `bytes` bytes that outlives the call: it
    /// is allocated on first use and replaced by a larger one only when a call needs more, so
    /// repeated calls neither allocate nor synchronise.  Every launch that uses it goes to
    /// this object's stream, which orders consecutive users; the smaller buffer a growth
    /// replaces is released with `hipFree`, which waits for the device first.
    pub fn with_workspace<R>(&self, bytes: usize, f: impl FnOnce(&mut HipSlice<u8>) -> CoreResult<R>)
                             -> CoreResult<R> {
        let mut guard = self.workspace.lock().map_err(|_| CoreError::Tensor("workspace lock poisoned".into()))?;
        if guard.as_ref().map_or(true, |w| w.len() < bytes) {
            *guard = None;  // free the smaller one first
            *guard = Some(HipSlice::<u8>::alloc(bytes.max(1), self.ordinal)?);
        }
        f(guard.as_mut().expect("workspace allocated above"))
    }

    /// mod.rs:196-225
    pub unsafe fn launch_rope<T: KvElement>(
        &self,
        x: &mut HipSlice<T>,
        cos_sin: &HipSlice<f32>,
        positions: &HipSlice<i32>,
        num_heads: i32,
        head_dim: i32,
        num_tokens: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_rope(x.as_mut_ptr(), cos_sin.as_ptr() as *const f32, positions.as_ptr() as *const i32,
                            num_heads, head_dim, num_tokens, T::DTYPE, self.stream))
    }

    /// mod.rs:227-262
    pub unsafe fn launch_reshape_and_cache<T: KvElement>(
        &self,
        k: &HipSlice<T>,
        v: &HipSlice<T>,
        k_cache: &mut HipSlice<T>,
        v_cache: &mut HipSlice<T>,
        slot_mapping: &HipSlice<i32>,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        batch_size: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_reshape_and_cache(k.as_ptr(), v.as_ptr(), k_cache.as_mut_ptr(), v_cache.as_mut_ptr(),
                                         slot_mapping.as_ptr() as *const i32, num_kv_heads, head_dim, block_size,
                                         batch_size, T::DTYPE, self.kv_block_stride, self.stream))
    }

    /// mod.rs:264-303
    pub unsafe fn launch_reshape_and_cache_isoquant<T: KvElement>(
        &self,
        k: &HipSlice<T>,
        v: &HipSlice<T>,
        k_cache: &mut HipSlice<T>,
        v_cache: &mut HipSlice<T>,
        slot_mapping: &HipSlice<i32>,
        rotation_metadata: &mut HipSlice<f32>,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        batch_size: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_reshape_and_cache_isoquant(
            k.as_ptr(), v.as_ptr(), k_cache.as_mut_ptr(), v_cache.as_mut_ptr(), slot_mapping.as_ptr() as *const i32,
            rotation_metadata.as_mut_ptr() as *mut f32, num_kv_heads, head_dim, block_size, batch_size, T::DTYPE,
            self.kv_block_stride, self.stream))
    }

    /// mod.rs:305-348 (no workspace: one workgroup per (sequence, kv-head) runs the whole
    /// context; `launch_v1_split` is the faster form).
    pub unsafe fn launch_v1<T: KvElement>(
        &self,
        query: &HipSlice<T>,
        key_cache: &HipSlice<T>,
        value_cache: &HipSlice<T>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        output: &mut HipSlice<T>,
        scale: f32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        max_blocks_per_seq: i32,
        batch_size: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_paged_attention_v1(
            query.as_ptr(), key_cache.as_ptr(), value_cache.as_ptr(), block_table.as_ptr() as *const i32,
            context_lens.as_ptr() as *const i32, output.as_mut_ptr(), scale, num_heads, num_kv_heads, head_dim,
            block_size, max_blocks_per_seq, batch_size, T::DTYPE, self.kv_block_stride, std::ptr::null_mut(), 0,
            self.stream))
    }

    /// mod.rs:350-399; `rotation_metadata` is accepted and ignored (identity rotation).
    pub unsafe fn launch_v1_plus<T: KvElement>(
        &self,
        query: &HipSlice<T>,
        key_cache: &HipSlice<T>,
        value_cache: &HipSlice<T>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        output: &mut HipSlice<T>,
        rotation_metadata: &HipSlice<f32>,
        scale: f32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        max_blocks_per_seq: i32,
        batch_size: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_paged_attention_v1_plus(
            query.as_ptr(), key_cache.as_ptr(), value_cache.as_ptr(), block_table.as_ptr() as *const i32,
            context_lens.as_ptr() as *const i32, output.as_mut_ptr(), rotation_metadata.as_ptr() as *const f32, scale,
            num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size, T::DTYPE,
            self.kv_block_stride, std::ptr::null_mut(), 0, self.stream))
    }

    /// mod.rs:401-456 (partition size 256).
    pub unsafe fn launch_v2_partition<T: KvElement>(
        &self,
        query: &HipSlice<T>,
        key_cache: &HipSlice<T>,
        value_cache: &HipSlice<T>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        tmp_out: &mut HipSlice<f32>,
        exp_sums: &mut HipSlice<f32>,
        max_logits: &mut HipSlice<f32>,
        rotation_metadata: &HipSlice<f32>,
        scale: f32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        max_blocks_per_seq: i32,
        num_partitions: i32,
        batch_size: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_paged_attention_v2_partition(
            query.as_ptr(), key_cache.as_ptr(), value_cache.as_ptr(), block_table.as_ptr() as *const i32,
            context_lens.as_ptr() as *const i32, tmp_out.as_mut_ptr() as *mut f32, exp_sums.as_mut_ptr() as *mut f32,
            max_logits.as_mut_ptr() as *mut f32, rotation_metadata.as_ptr() as *const f32, scale, num_heads,
            num_kv_heads, head_dim, block_size, max_blocks_per_seq, num_partitions, batch_size, V2_PARTITION_SIZE,
            T::DTYPE, self.kv_block_stride, self.stream))
    }

    /// mod.rs:458-508 (partition size 256; no 512-partition cap).
    pub unsafe fn launch_v2_reduce<T: KvElement>(
        &self,
        output: &mut HipSlice<T>,
        exp_sums: &HipSlice<f32>,
        max_logits: &HipSlice<f32>,
        tmp_out: &HipSlice<f32>,
        context_lens: &HipSlice<i32>,
        rotation_metadata: &HipSlice<f32>,
        num_heads: i32,
        head_dim: i32,
        num_partitions: i32,
        batch_size: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_paged_attention_v2_reduce(
            output.as_mut_ptr(), exp_sums.as_ptr() as *const f32, max_logits.as_ptr() as *const f32,
            tmp_out.as_ptr() as *const f32, context_lens.as_ptr() as *const i32,
            rotation_metadata.as_ptr() as *const f32, num_heads, head_dim, num_partitions, batch_size,
            V2_PARTITION_SIZE, T::DTYPE, self.stream))
    }

    // ---------------------------------------------------------- entries beyond mod.rs --

    /// Workspace bytes of `launch_v1_split` (0: none needed).
    pub fn v1_workspace_bytes(&self, batch_size: i32, num_heads: i32, num_kv_heads: i32, head_dim: i32,
                              block_size: i32, max_blocks_per_seq: i32) -> usize {
        // SAFETY: pure size query.
        unsafe {
            ffi::rg_paged_attention_v1_workspace_bytes(batch_size, num_heads, num_kv_heads, head_dim, block_size,
                                                       max_blocks_per_seq)
        }
    }

    /// Bytes of the v2 scratch (tmp_out, exp_sums, max_logits) for `num_partitions` partitions.
    pub fn v2_workspace_bytes(&self, batch_size: i32, num_heads: i32, num_partitions: i32, head_dim: i32) -> usize {
        // SAFETY: pure size query.
        unsafe { ffi::rg_v2_workspace_bytes(batch_size, num_heads, num_partitions, head_dim) }
    }

    /// `launch_v1_plus` with a workspace: the KV blocks of the whole batch split evenly over
    /// every compute unit, partials merged by a second kernel (the fast path).
    pub unsafe fn launch_v1_split<T: KvElement>(
        &self,
        query: &HipSlice<T>,
        key_cache: &HipSlice<T>,
        value_cache: &HipSlice<T>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        output: &mut HipSlice<T>,
        scale: f32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        max_blocks_per_seq: i32,
        batch_size: i32,
        workspace: &mut HipSlice<u8>,
    ) -> CoreResult<()> {
        status(ffi::rg_paged_attention_v1(
            query.as_ptr(), key_cache.as_ptr(), value_cache.as_ptr(), block_table.as_ptr() as *const i32,
            context_lens.as_ptr() as *const i32, output.as_mut_ptr(), scale, num_heads, num_kv_heads, head_dim,
            block_size, max_blocks_per_seq, batch_size, T::DTYPE, self.kv_block_stride, workspace.as_mut_ptr(),
            workspace.len(), self.stream))
    }

    /// One decode step's RoPE + cache write (one new token per sequence: `key` / `value`
    /// [batch, H_kv, D]) and `launch_v1_split` in the stream-K decode's launches: the same
    /// output and caches as `launch_rope_reshape_and_cache` followed by `launch_v1_split`,
    /// with `query` left unrotated.  `slot_mapping[s]` is -1 or the slot of position
    /// `context_lens[s] - 1` in sequence s's block table.
    pub unsafe fn launch_rope_reshape_and_cache_v1<T: KvElement>(
        &self,
        query: &HipSlice<T>,
        key: &HipSlice<T>,
        value: &HipSlice<T>,
        key_cache: &mut HipSlice<T>,
        value_cache: &mut HipSlice<T>,
        cos_sin: &HipSlice<f32>,
        positions: &HipSlice<i32>,
        slot_mapping: &HipSlice<i32>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        output: &mut HipSlice<T>,
        scale: f32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        max_blocks_per_seq: i32,
        batch_size: i32,
        workspace: &mut HipSlice<u8>,
    ) -> CoreResult<()> {
        status(ffi::rg_rope_reshape_and_cache_paged_attention_v1(
            query.as_ptr(), key.as_ptr(), value.as_ptr(), key_cache.as_mut_ptr(), value_cache.as_mut_ptr(),
            cos_sin.as_ptr() as *const f32, positions.as_ptr() as *const i32, slot_mapping.as_ptr() as *const i32,
            block_table.as_ptr() as *const i32, context_lens.as_ptr() as *const i32, output.as_mut_ptr(), scale,
            num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size, T::DTYPE,
            self.kv_block_stride, workspace.as_mut_ptr(), workspace.len(), self.stream))
    }

    /// `launch_v1_split` on the library's static per-device scratch: no allocation anywhere,
    /// for code under graph capture or loops that cannot allocate.  Calls overlapping in time
    /// on one device race on that scratch.
    pub unsafe fn launch_v1_no_alloc<T: KvElement>(
        &self,
        query: &HipSlice<T>,
        key_cache: &HipSlice<T>,
        value_cache: &HipSlice<T>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        output: &mut HipSlice<T>,
        scale: f32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        max_blocks_per_seq: i32,
        batch_size: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_paged_attention_v1_no_alloc(
            query.as_ptr(), key_cache.as_ptr(), value_cache.as_ptr(), block_table.as_ptr() as *const i32,
            context_lens.as_ptr() as *const i32, output.as_mut_ptr(), scale, num_heads, num_kv_heads, head_dim,
            block_size, max_blocks_per_seq, batch_size, T::DTYPE, self.kv_block_stride, self.stream))
    }

    /// The v2 computation in one call (paged_attn_op.rs:108-158): with a workspace of at least
    /// max(v2_workspace_bytes, v1_workspace_bytes) the balanced split-K form runs.
    pub unsafe fn launch_v2<T: KvElement>(
        &self,
        query: &HipSlice<T>,
        key_cache: &HipSlice<T>,
        value_cache: &HipSlice<T>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        output: &mut HipSlice<T>,
        scale: f32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        max_blocks_per_seq: i32,
        batch_size: i32,
        max_context_len: i32,
        partition_size: i32,
        workspace: &mut HipSlice<u8>,
    ) -> CoreResult<()> {
        status(ffi::rg_paged_attention_v2(
            query.as_ptr(), key_cache.as_ptr(), value_cache.as_ptr(), block_table.as_ptr() as *const i32,
            context_lens.as_ptr() as *const i32, output.as_mut_ptr(), scale, num_heads, num_kv_heads, head_dim,
            block_size, max_blocks_per_seq, batch_size, max_context_len, partition_size, T::DTYPE,
            self.kv_block_stride, workspace.as_mut_ptr(), workspace.len(), self.stream))
    }

    /// RoPE on q (in place) and k, then the cache write, one pass over the new tokens.
    pub unsafe fn launch_rope_reshape_and_cache<T: KvElement>(
        &self,
        q: &mut HipSlice<T>,
        k: &HipSlice<T>,
        v: &HipSlice<T>,
        k_cache: &mut HipSlice<T>,
        v_cache: &mut HipSlice<T>,
        cos_sin: &HipSlice<f32>,
        positions: &HipSlice<i32>,
        slot_mapping: &HipSlice<i32>,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        num_tokens: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_rope_reshape_and_cache(
            q.as_mut_ptr(), k.as_ptr(), v.as_ptr(), k_cache.as_mut_ptr(), v_cache.as_mut_ptr(),
            cos_sin.as_ptr() as *const f32, positions.as_ptr() as *const i32, slot_mapping.as_ptr() as *const i32,
            num_heads, num_kv_heads, head_dim, block_size, num_tokens, T::DTYPE, self.kv_block_stride, self.stream))
    }

    /// The same reading q/k/v from one fused projection output `qkv` (`qkv_token_stride`
    /// elements per token); rotated q goes to `q_out`.
    pub unsafe fn launch_qkv_rope_reshape_and_cache<T: KvElement>(
        &self,
        qkv: &HipSlice<T>,
        qkv_token_stride: i64,
        q_out: &mut HipSlice<T>,
        k_cache: &mut HipSlice<T>,
        v_cache: &mut HipSlice<T>,
        cos_sin: &HipSlice<f32>,
        positions: &HipSlice<i32>,
        slot_mapping: &HipSlice<i32>,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        num_tokens: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_qkv_rope_reshape_and_cache(
            qkv.as_ptr(), qkv_token_stride, q_out.as_mut_ptr(), k_cache.as_mut_ptr(), v_cache.as_mut_ptr(),
            cos_sin.as_ptr() as *const f32, positions.as_ptr() as *const i32, slot_mapping.as_ptr() as *const i32,
            num_heads, num_kv_heads, head_dim, block_size, num_tokens, T::DTYPE, self.kv_block_stride, self.stream))
    }

    /// The fused q/k/v projection and launch_qkv_rope_reshape_and_cache in one pass for decode
    /// batches (num_tokens <= 128, head_dim 32 or 64); q_out rows of num_heads * head_dim.
    pub unsafe fn launch_linear_qkv_rope_reshape_and_cache<T: KvElement>(
        &self,
        x: &HipSlice<T>,
        weight_qkv: &HipSlice<T>,
        q_out: &mut HipSlice<T>,
        k_cache: &mut HipSlice<T>,
        v_cache: &mut HipSlice<T>,
        cos_sin: &HipSlice<f32>,
        positions: &HipSlice<i32>,
        slot_mapping: &HipSlice<i32>,
        num_tokens: i32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        in_features: i32,
        x_row_stride: i64,
    ) -> CoreResult<()> {
        status(ffi::rg_linear_qkv_rope_reshape_and_cache(
            x.as_ptr(), weight_qkv.as_ptr(), q_out.as_mut_ptr(), k_cache.as_mut_ptr(), v_cache.as_mut_ptr(),
            cos_sin.as_ptr() as *const f32, positions.as_ptr() as *const i32, slot_mapping.as_ptr() as *const i32,
            num_tokens, num_heads, num_kv_heads, head_dim, block_size, in_features, x_row_stride,
            in_features as i64, (num_heads * head_dim) as i64, self.kv_block_stride, T::DTYPE, self.stream))
    }

    /// Packed causal prefill of `num_seqs` sequences (rows `cu_seqlens[s] .. cu_seqlens[s+1]`)
    /// over the paged cache.
    pub unsafe fn launch_prefill_packed<T: KvElement>(
        &self,
        query: &HipSlice<T>,
        key_cache: &HipSlice<T>,
        value_cache: &HipSlice<T>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        cu_seqlens: &HipSlice<i32>,
        output: &mut HipSlice<T>,
        scale: f32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        max_blocks_per_seq: i32,
        num_seqs: i32,
        num_tokens: i32,
        max_query_len: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_prefill_packed(
            query.as_ptr(), key_cache.as_ptr(), value_cache.as_ptr(), block_table.as_ptr() as *const i32,
            context_lens.as_ptr() as *const i32, cu_seqlens.as_ptr() as *const i32, output.as_mut_ptr(), scale,
            num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, num_seqs, num_tokens, max_query_len,
            T::DTYPE, self.kv_block_stride, self.stream))
    }

    /// Whole-block copies between pools on the device and/or in pinned host memory, every
    /// layer in one launch (the data movement behind swap_out / swap_in / fork).
    pub unsafe fn launch_copy_blocks(
        &self,
        src_pool: *const c_void,
        dst_pool: *mut c_void,
        block_mapping: &HipSlice<i32>,
        num_pairs: i32,
        block_bytes: i64,
        src_block_stride_bytes: i64,
        dst_block_stride_bytes: i64,
        num_layers: i32,
        src_layer_stride_bytes: i64,
        dst_layer_stride_bytes: i64,
    ) -> CoreResult<()> {
        status(ffi::rg_copy_blocks(src_pool, dst_pool, block_mapping.as_ptr() as *const i32, num_pairs, block_bytes,
                                   src_block_stride_bytes, dst_block_stride_bytes, num_layers,
                                   src_layer_stride_bytes, dst_layer_stride_bytes, self.stream))
    }

    /// Residual add + RMSNorm over `num_rows` rows (`residual` may be None).
    pub unsafe fn launch_rms_norm<T: KvElement>(
        &self,
        x: &HipSlice<T>,
        residual: Option<&mut HipSlice<T>>,
        weight: &HipSlice<T>,
        out: &mut HipSlice<T>,
        eps: f32,
        num_rows: i32,
        hidden_size: i32,
    ) -> CoreResult<()> {
        let r = residual.map_or(std::ptr::null_mut(), |r| r.as_mut_ptr());
        status(ffi::rg_rms_norm(x.as_ptr(), r, weight.as_ptr(), out.as_mut_ptr(), eps, num_rows, hidden_size,
                                T::DTYPE, self.stream))
    }

    /// Opt-in check (no counterpart in mod.rs): every context length within its table row and
    /// every block number the contexts use within the pool; synchronises the stream and names
    /// the first bad entry in the error.
    pub unsafe fn validate_block_tables(
        &self,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        batch_size: i32,
        max_blocks_per_seq: i32,
        block_size: i32,
        num_blocks: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_validate_block_tables(block_table.as_ptr(), context_lens.as_ptr(), batch_size,
                                             max_blocks_per_seq, block_size, num_blocks, self.stream))
    }

    /// Opt-in check of a slot mapping against a pool of `num_slots` slots (negative slots are padding).
    pub unsafe fn validate_slot_mapping(&self, slot_mapping: &HipSlice<i32>, num_tokens: i32, num_slots: i64)
        -> CoreResult<()> {
        status(ffi::rg_validate_slot_mapping(slot_mapping.as_ptr(), num_tokens, num_slots, self.stream))
    }

    /// out [num_rows, intermediate_size] = silu(x . gate^T) * (x . up^T) with the gate and up rows of
    /// `weight_gate_up` interleaved in blocks of 16 (see the header), decode batches only.
    pub unsafe fn launch_linear_silu_mul<T: KvElement>(
        &self,
        x: &HipSlice<T>,
        weight_gate_up: &HipSlice<T>,
        out: &mut HipSlice<T>,
        num_rows: i32,
        intermediate_size: i32,
        in_features: i32,
        x_row_stride: i64,
        weight_row_stride: i64,
        out_row_stride: i64,
    ) -> CoreResult<()> {
        status(ffi::rg_linear_silu_mul(x.as_ptr(), weight_gate_up.as_ptr(), out.as_mut_ptr(), num_rows,
                                       intermediate_size, in_features, x_row_stride, weight_row_stride,
                                       out_row_stride, T::DTYPE, self.stream))
    }

    /// Split-K workspace bytes of launch_linear for this shape on the current device.
    pub fn linear_workspace_bytes(&self, num_rows: i32, out_features: i32, in_features: i32) -> usize {
        // SAFETY: a pure size computation.
        unsafe { ffi::rg_linear_workspace_bytes(num_rows, out_features, in_features) }
    }

    /// out [num_rows, out_features] = x [num_rows, in_features] . weight^T for decode batches
    /// (num_rows <= 128); row strides in elements.  With a workspace of linear_workspace_bytes
    /// narrow or deep layers split K over more workgroups.
    pub unsafe fn launch_linear<T: KvElement>(
        &self,
        x: &HipSlice<T>,
        weight: &HipSlice<T>,
        out: &mut HipSlice<T>,
        num_rows: i32,
        out_features: i32,
        in_features: i32,
        x_row_stride: i64,
        weight_row_stride: i64,
        out_row_stride: i64,
        workspace: Option<&mut HipSlice<u8>>,
    ) -> CoreResult<()> {
        let (ws, ws_len) = workspace.map_or((std::ptr::null_mut(), 0), |w| (w.as_mut_ptr(), w.len()));
        status(ffi::rg_linear(x.as_ptr(), weight.as_ptr(), out.as_mut_ptr(), num_rows, out_features, in_features,
                              x_row_stride, weight_row_stride, out_row_stride, ws, ws_len, T::DTYPE, self.stream))
    }

    /// residual [num_rows, out_features] += x . weight^T, rounded as launch_linear followed by
    /// the residual add of launch_rms_norm; the workspace as for launch_linear.
    pub unsafe fn launch_linear_residual<T: KvElement>(
        &self,
        x: &HipSlice<T>,
        weight: &HipSlice<T>,
        residual: &mut HipSlice<T>,
        num_rows: i32,
        out_features: i32,
        in_features: i32,
        x_row_stride: i64,
        weight_row_stride: i64,
        residual_row_stride: i64,
        workspace: Option<&mut HipSlice<u8>>,
    ) -> CoreResult<()> {
        let (ws, ws_len) = workspace.map_or((std::ptr::null_mut(), 0), |w| (w.as_mut_ptr(), w.len()));
        status(ffi::rg_linear_residual(x.as_ptr(), weight.as_ptr(), residual.as_mut_ptr(), num_rows, out_features,
                                       in_features, x_row_stride, weight_row_stride, residual_row_stride, ws, ws_len,
                                       T::DTYPE, self.stream))
    }

    /// launch_linear_silu_mul on the RmsNorm of the residual stream x (norm weight [in_features]).
    pub unsafe fn launch_rms_norm_linear_silu_mul<T: KvElement>(
        &self,
        x: &HipSlice<T>,
        norm_weight: &HipSlice<T>,
        eps: f32,
        weight_gate_up: &HipSlice<T>,
        out: &mut HipSlice<T>,
        num_rows: i32,
        intermediate_size: i32,
        in_features: i32,
        x_row_stride: i64,
    ) -> CoreResult<()> {
        status(ffi::rg_rms_norm_linear_silu_mul(x.as_ptr(), norm_weight.as_ptr(), eps, weight_gate_up.as_ptr(),
                                                out.as_mut_ptr(), num_rows, intermediate_size, in_features,
                                                x_row_stride, in_features as i64, intermediate_size as i64,
                                                T::DTYPE, self.stream))
    }

    /// launch_linear_qkv_rope_reshape_and_cache on the RmsNorm of the residual stream x.
    pub unsafe fn launch_rms_norm_linear_qkv_rope_reshape_and_cache<T: KvElement>(
        &self,
        x: &HipSlice<T>,
        norm_weight: &HipSlice<T>,
        eps: f32,
        weight_qkv: &HipSlice<T>,
        q_out: &mut HipSlice<T>,
        k_cache: &mut HipSlice<T>,
        v_cache: &mut HipSlice<T>,
        cos_sin: &HipSlice<f32>,
        positions: &HipSlice<i32>,
        slot_mapping: &HipSlice<i32>,
        num_tokens: i32,
        num_heads: i32,
        num_kv_heads: i32,
        head_dim: i32,
        block_size: i32,
        in_features: i32,
        x_row_stride: i64,
    ) -> CoreResult<()> {
        status(ffi::rg_rms_norm_linear_qkv_rope_reshape_and_cache(
            x.as_ptr(), norm_weight.as_ptr(), eps, weight_qkv.as_ptr(), q_out.as_mut_ptr(), k_cache.as_mut_ptr(),
            v_cache.as_mut_ptr(), cos_sin.as_ptr() as *const f32, positions.as_ptr() as *const i32,
            slot_mapping.as_ptr() as *const i32, num_tokens, num_heads, num_kv_heads, head_dim, block_size,
            in_features, x_row_stride, in_features as i64, (num_heads * head_dim) as i64, self.kv_block_stride,
            T::DTYPE, self.stream))
    }

    /// out = silu(gate) * up over the fused gate/up projection output.
    pub unsafe fn launch_silu_and_mul<T: KvElement>(
        &self,
        gate_up: &HipSlice<T>,
        out: &mut HipSlice<T>,
        num_rows: i32,
        intermediate_size: i32,
    ) -> CoreResult<()> {
        status(ffi::rg_silu_and_mul(gate_up.as_ptr(), out.as_mut_ptr(), num_rows, intermediate_size, T::DTYPE,
                                    self.stream))
    }
}

/// Host-side cos/sin table [max_position, head_dim] for RoPE (HF Llama convention).
pub fn rope_cos_sin_table(max_position: i32, head_dim: i32, theta: f64) -> CoreResult<Vec<f32>> {
    let mut table = vec![0f32; (max_position.max(0) as usize) * (head_dim.max(0) as usize)];
    // SAFETY: the table holds max_position * head_dim floats.
    status(unsafe { ffi::rg_rope_cos_sin_table(table.as_mut_ptr(), max_position, head_dim, theta) })?;
    Ok(table)
}
