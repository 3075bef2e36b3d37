//! vllm-hip: Railgun's attention hot path on AMD Instinct MI355X (gfx950).
//!
//! The HIP counterpart of crates/vllm-cuda's kernel module: `PagedAttentionKernels` and
//! `PagedAttentionOp` with the method names, argument order and errors of
//! crates/vllm-cuda/src/kernels/mod.rs:23-509 and paged_attn_op.rs:12-269, calling the
//! hand-written gfx950 kernels of librailgun_hip.so through its C ABI (`ffi`).

pub mod buffer;
pub mod ffi;
pub mod hip;
pub mod kernels;
pub mod op;

pub use buffer::{Bf16, HipSlice, KvElement, F16};
pub use kernels::{last_error, rope_cos_sin_table, status, PagedAttentionKernels};
pub use op::PagedAttentionOp;
