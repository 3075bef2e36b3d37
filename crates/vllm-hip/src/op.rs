//! `PagedAttentionOp` on HIP: crates/vllm-cuda/src/kernels/paged_attn_op.rs:12-269 with the
//! same fields, methods and dispatch.  Shapes come from the buffers' lengths and the op's
//! head counts (the reference reads them from candle tensors, :63-65):
//! q is [batch, num_heads, head_dim], block_table [batch, max_blocks], k/v
//! [tokens, num_kv_heads, head_dim], x [tokens, heads, head_dim], positions [tokens].

use std::sync::Arc;

use vllm_core::{CoreError, Result as CoreResult};

use crate::buffer::{HipSlice, KvElement};
use crate::kernels::PagedAttentionKernels;

/// Contexts up to this length run v1+ (paged_attn_op.rs:89), longer ones v2.
pub const V1_MAX_CONTEXT: usize = 4096;
/// Partition size of execute's v2 branch (any multiple of the block size gives the same result).
pub const EXECUTE_V2_PARTITION: usize = 512;

/// The PagedAttention custom operation (paged_attn_op.rs:12-19).
pub struct PagedAttentionOp {
    pub scale: f32,
    pub num_heads: usize,
    pub num_kv_heads: usize,
    pub head_dim: usize,
    pub block_size: usize,
    pub kernels: Arc<PagedAttentionKernels>,
}

fn shape_err(what: &str) -> CoreError {
    CoreError::Tensor(format!("PagedAttentionOp: {what}"))
}

impl PagedAttentionOp {
    /// paged_attn_op.rs:45-166: q [batch, num_heads, head_dim] -> a new output of the same
    /// shape (zero-filled first, as :86 does).  `max_context_len <= 4096` runs v1+ split over
    /// every compute unit, longer runs the v2 split-K form.  Their scratch is the kernels'
    /// grow-only workspace (`PagedAttentionKernels::with_workspace`), not an allocation per
    /// call as the reference's v2 scratch is (:113-123): the call only queues work on the
    /// kernels' stream and returns without waiting for it.
    pub fn execute<T: KvElement>(
        &self,
        q: &HipSlice<T>,
        k_cache: &HipSlice<T>,
        v_cache: &HipSlice<T>,
        block_table: &HipSlice<i32>,
        context_lens: &HipSlice<i32>,
        rotation_metadata: &HipSlice<f32>,
        max_context_len: usize,
    ) -> CoreResult<HipSlice<T>> {
        if self.head_dim % 4 != 0 {
            return Err(CoreError::NotSupported {
                feature: "PagedAttention",
                reason: format!("Head dimension ({}) must be a multiple of 4 for IsoQuant.", self.head_dim),
            });
        }
        let row = self.num_heads * self.head_dim;
        if q.len() % row != 0 {
            return Err(shape_err("q is not [batch, num_heads, head_dim]"));
        }
        let batch = q.len() / row;
        if batch == 0 {
            return HipSlice::zeros(0, self.kernels.ordinal(), self.kernels.stream());
        }
        if context_lens.len() != batch || block_table.len() % batch != 0 {
            return Err(shape_err("context_lens must be [batch] and block_table [batch, max_blocks]"));
        }
        let max_blocks = block_table.len() / batch;
        let k = &self.kernels;
        let mut out = HipSlice::<T>::zeros(q.len(), k.ordinal(), k.stream())?;
        let (h, hkv, d, bs) = (self.num_heads as i32, self.num_kv_heads as i32, self.head_dim as i32,
                               self.block_size as i32);
        let v1_ws = k.v1_workspace_bytes(batch as i32, h, hkv, d, bs, max_blocks as i32);
        let _ = rotation_metadata;  // identity rotation
        if max_context_len <= V1_MAX_CONTEXT {
            k.with_workspace(v1_ws, |ws| {
                // SAFETY: shapes checked above; indices are the caller's responsibility, as in
                // the reference.
                unsafe {
                    k.launch_v1_split(q, k_cache, v_cache, block_table, context_lens, &mut out, self.scale, h, hkv,
                                      d, bs, max_blocks as i32, batch as i32, ws)
                }
            })?;
        } else {
            let parts = (max_context_len + EXECUTE_V2_PARTITION - 1) / EXECUTE_V2_PARTITION;
            let bytes = k.v2_workspace_bytes(batch as i32, h, parts as i32, d).max(v1_ws);
            k.with_workspace(bytes, |ws| {
                // SAFETY: as above.
                unsafe {
                    k.launch_v2(q, k_cache, v_cache, block_table, context_lens, &mut out, self.scale, h, hkv, d, bs,
                                max_blocks as i32, batch as i32, max_context_len as i32,
                                EXECUTE_V2_PARTITION as i32, ws)
                }
            })?;
        }
        Ok(out)
    }

    /// paged_attn_op.rs:168-233: k, v [tokens, num_kv_heads, head_dim] into the caches, in
    /// place (the reference writes into clones of the cache slices, defect D2).
    pub fn reshape_and_cache<T: KvElement>(
        &self,
        k: &HipSlice<T>,
        v: &HipSlice<T>,
        k_cache: &mut HipSlice<T>,
        v_cache: &mut HipSlice<T>,
        slot_mapping: &HipSlice<i32>,
        rotation_metadata: &mut HipSlice<f32>,
        use_isoquant: bool,
    ) -> CoreResult<()> {
        let row = self.num_kv_heads * self.head_dim;
        if k.len() % row != 0 || v.len() != k.len() {
            return Err(shape_err("k and v must be [tokens, num_kv_heads, head_dim]"));
        }
        let tokens = (k.len() / row) as i32;
        if slot_mapping.len() != tokens as usize {
            return Err(shape_err("slot_mapping must be [tokens]"));
        }
        let (hkv, d, bs) = (self.num_kv_heads as i32, self.head_dim as i32, self.block_size as i32);
        // SAFETY: shapes checked; slots are the caller's responsibility, as in the reference.
        unsafe {
            if use_isoquant {
                self.kernels.launch_reshape_and_cache_isoquant(k, v, k_cache, v_cache, slot_mapping,
                                                               rotation_metadata, hkv, d, bs, tokens)
            } else {
                self.kernels.launch_reshape_and_cache(k, v, k_cache, v_cache, slot_mapping, hkv, d, bs, tokens)
            }
        }
    }

    /// paged_attn_op.rs:236-268: RoPE in place on x [tokens, heads, head_dim].
    pub fn apply_rope<T: KvElement>(
        &self,
        x: &mut HipSlice<T>,
        cos_sin: &HipSlice<f32>,
        positions: &HipSlice<i32>,
    ) -> CoreResult<()> {
        let tokens = positions.len();
        if tokens == 0 {
            return Ok(());
        }
        if x.len() % (tokens * self.head_dim) != 0 {
            return Err(shape_err("x must be [tokens, heads, head_dim] with one position per token"));
        }
        let heads = (x.len() / (tokens * self.head_dim)) as i32;
        // SAFETY: shapes checked; positions index cos_sin, the caller's responsibility.
        unsafe { self.kernels.launch_rope(x, cos_sin, positions, heads, self.head_dim as i32, tokens as i32) }
    }
}
