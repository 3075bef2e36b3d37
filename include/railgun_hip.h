/*
 * railgun_hip.h — C ABI of the MI355X (gfx950) attention hot path.
 *
 * Every entry point is `extern "C"`, takes raw device pointers and plain
 * integers, launches asynchronously on the HIP stream it is given (NULL =
 * the null stream) and never allocates device memory.  This is the surface a
 * Rust FFI crate binds in place of Railgun's `PagedAttentionKernels`
 * (crates/vllm-cuda/src/kernels/mod.rs:23-509); the comment above each entry
 * names the launcher it replaces.
 *
 * Conventions shared by all entries
 *  - Return value: RG_OK (0) or one of the RG_ERR_* codes below.  On error
 *    rg_last_error() returns a thread-local, human-readable message.  Argument
 *    checks mirror the reference's CoreError::NotSupported / CoreError::Tensor
 *    (crates/vllm-cuda/src/kernels/mod.rs:42-54,477-482).
 *  - dtype: RG_DTYPE_F32 / RG_DTYPE_BF16 / RG_DTYPE_F16, the element type of
 *    q/k/v/output and of the KV cache.  Arithmetic is fp32 throughout.
 *  - KV cache layout per block: [num_kv_heads, block_size, head_dim]
 *    (crates/vllm-cuda/src/kernels/paged_attention.cu:9-10).  kv_block_stride
 *    is the distance in ELEMENTS between consecutive blocks; pass 0 for the
 *    dense layout (num_kv_heads*block_size*head_dim).  Railgun's fused pool
 *    [num_blocks, 2, num_kv_heads, block_size, head_dim]
 *    (crates/vllm-paged-attention/src/block.rs:70) is addressed with
 *    k_cache = base, v_cache = base + num_kv_heads*block_size*head_dim and
 *    kv_block_stride = 2*num_kv_heads*block_size*head_dim.
 *  - block_table is row-major int32 [batch, max_blocks_per_seq]; context_lens
 *    is int32 [batch]; slot_mapping is int32 [num_tokens] with
 *    slot = block_id*block_size + position%block_size, negative = skip
 *    (crates/vllm-scheduler/src/scheduler.rs:230-235,258-263).
 *  - Grouped-query attention: q-head h reads kv-head h / (num_heads/num_kv_heads)
 *    (crates/vllm-cuda/src/kernels/paged_attention.cu:40).
 *  - rotation_metadata arguments exist for signature compatibility with the
 *    IsoQuant launchers.  Railgun's rotation is the identity
 *    (crates/vllm-cuda/src/kernels/isoquant_utils.cuh:54-58), so the attention
 *    entries ignore it (it may be NULL).
 */
#ifndef RAILGUN_HIP_H
#define RAILGUN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RG_ABI_VERSION 1

/* Status codes. */
#define RG_OK 0
#define RG_ERR_INVALID_ARGUMENT 1 /* null pointer, negative size, bad GQA ratio  */
#define RG_ERR_NOT_SUPPORTED 2    /* head_dim / dtype / block_size out of range  */
#define RG_ERR_HIP 3              /* HIP runtime or launch failure               */
#define RG_ERR_WORKSPACE 4        /* workspace missing or smaller than required  */

/* Element types. */
#define RG_DTYPE_F32 0
#define RG_DTYPE_BF16 1
#define RG_DTYPE_F16 2

/* Largest head_dim the paged-attention entries accept
 * (MAX_HEAD_DIM_PAGED_ATTENTION, crates/vllm-cuda/src/kernels/mod.rs:20). */
#define RG_MAX_HEAD_DIM 256

/* Thread-local message describing the last failing call on this thread. */
const char* rg_last_error(void);

/* RG_ABI_VERSION of the loaded library. */
int rg_abi_version(void);

/* Checks that `device_ordinal` is a gfx950 device and that every kernel's code
 * object is loadable there.  Replaces PagedAttentionKernels::new
 * (crates/vllm-cuda/src/kernels/mod.rs:57-190), which loads the PTX modules;
 * here the code objects are linked into the library, so nothing is cached
 * and the call is optional. */
int rg_init(int device_ordinal);

/* ---------------------------------------------------------------- RoPE ---- */

/* In-place rotate-half RoPE on x [num_tokens, num_heads, head_dim]:
 *   x[i]      = x[i]*c - x[i+D/2]*s
 *   x[i+D/2]  = x[i+D/2]*c + x[i]*s,   c = cos_sin[pos*D + i], s = cos_sin[pos*D + D/2 + i]
 * with pos = positions[token].  cos_sin is fp32 [max_position, head_dim].
 * Replaces launch_rope (crates/vllm-cuda/src/kernels/mod.rs:196-225) /
 * rotary_embedding_kernel (crates/vllm-cuda/src/kernels/rope.cu:11-42). */
int rg_rope(void* x, const float* cos_sin, const int32_t* positions,
            int32_t num_heads, int32_t head_dim, int32_t num_tokens,
            int32_t dtype, void* stream);

/* Host helper (no GPU): fills `table` (host memory, fp32 [max_position, head_dim])
 * with the HF Llama convention inv_freq_i = theta^(-2i/D), angle = pos*inv_freq_i,
 * cos in columns [0, D/2), sin in columns [D/2, D).  Computed in double and
 * rounded once to fp32.  The reference never builds this table
 * (crates/vllm-cuda/src/kernels/paged_attn_op.rs:236-268 takes it as input). */
int rg_rope_cos_sin_table(float* table, int32_t max_position, int32_t head_dim,
                          double theta);

/* ------------------------------------------------------ KV-cache writes ---- */

/* Scatters k, v [num_tokens, num_kv_heads, head_dim] into the paged caches:
 * slot = slot_mapping[t]; skipped when slot < 0; block = slot / block_size,
 * offset = slot % block_size.  A bit-exact copy.
 * Replaces launch_reshape_and_cache (crates/vllm-cuda/src/kernels/mod.rs:227-262)
 * / reshape_and_cache (crates/vllm-cuda/src/kernels/paged_attention.cu:111-138). */
int rg_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                         const int32_t* slot_mapping, int32_t num_kv_heads,
                         int32_t head_dim, int32_t block_size, int32_t num_tokens,
                         int32_t dtype, int64_t kv_block_stride, void* stream);

/* As rg_reshape_and_cache, and additionally, for every token written at
 * offset 0 of its block, stores the identity rotation (0,0,0,1, 0,0,0,1) into
 * rotation_metadata fp32 [num_blocks, num_kv_heads, head_dim/4, 8].  The
 * K/V data are copied unchanged (the rotation is the identity).
 * Replaces launch_reshape_and_cache_isoquant
 * (crates/vllm-cuda/src/kernels/mod.rs:264-303) /
 * reshape_and_cache_isoquant (crates/vllm-cuda/src/kernels/paged_attention.cu:140-185). */
int rg_reshape_and_cache_isoquant(const void* k, const void* v, void* k_cache,
                                  void* v_cache, const int32_t* slot_mapping,
                                  float* rotation_metadata, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t block_size,
                                  int32_t num_tokens, int32_t dtype,
                                  int64_t kv_block_stride, void* stream);

/* One pass over the new tokens: RoPE on q [num_tokens, num_heads, head_dim]
 * in place, RoPE on k [num_tokens, num_kv_heads, head_dim] (k itself is left
 * unchanged; the rotated rows go to the cache) and the scatter of rotated k
 * and of v into the paged caches by slot_mapping, with the same arithmetic
 * as rg_rope followed by rg_reshape_and_cache.  New entry (the reference's
 * RoPE has no caller, crates/vllm-cuda/src/kernels/paged_attn_op.rs:236-268). */
int rg_rope_reshape_and_cache(void* q, const void* k, const void* v,
                              void* k_cache, void* v_cache, const float* cos_sin,
                              const int32_t* positions, const int32_t* slot_mapping,
                              int32_t num_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t block_size,
                              int32_t num_tokens, int32_t dtype,
                              int64_t kv_block_stride, void* stream);

/* rg_rope_reshape_and_cache for the output of one fused q/k/v projection:
 * token t's q, k and v rows are read from qkv + t*qkv_token_stride at
 * columns [0, H*D), [H*D, (H+H_kv)*D) and [(H+H_kv)*D, (H+2*H_kv)*D)
 * (qkv_token_stride >= (H+2*H_kv)*D elements); the rotated q rows are
 * written to q_out [num_tokens, num_heads, head_dim] (qkv is not modified),
 * rotated k and v go to the paged caches as in rg_rope_reshape_and_cache.
 * Same arithmetic, one pass.  New entry: it serves the decode step of a model
 * whose q/k/v projections are one GEMM (the reference projects q, k and v
 * separately and never applies RoPE,
 * crates/vllm-models/src/llama/attention.rs:104-125). */
int rg_qkv_rope_reshape_and_cache(const void* qkv, int64_t qkv_token_stride,
                                  void* q_out, void* k_cache, void* v_cache,
                                  const float* cos_sin, const int32_t* positions,
                                  const int32_t* slot_mapping, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim,
                                  int32_t block_size, int32_t num_tokens,
                                  int32_t dtype, int64_t kv_block_stride,
                                  void* stream);

/* Copies whole KV blocks between two pools: for i < num_pairs and every layer
 * l < num_layers, the block_bytes bytes at
 *   src_pool + l*src_layer_stride_bytes + block_mapping[2i]*src_block_stride_bytes
 * go to
 *   dst_pool + l*dst_layer_stride_bytes + block_mapping[2i+1]*dst_block_stride_bytes.
 * A bit-exact copy.  The pools may be device memory or device-accessible pinned host
 * memory (hipHostMalloc), so one entry serves GPU -> CPU swap-out, CPU -> GPU swap-in and
 * GPU -> GPU copy-on-write; block_mapping must be device-accessible too.  Sizes and
 * strides are multiples of 16 bytes, pools 16-byte aligned; destinations must not overlap
 * each other or the sources.  With Railgun's fused pool [NB, 2, H_kv, bs, D] one block
 * (K and V) is contiguous: block_bytes = stride = 2*H_kv*bs*D*elem.  New entry: the
 * reference's swap_out / swap_in move block ids between free lists but copy no data
 * (crates/vllm-paged-attention/src/allocator.rs:102-153, "TODO ... physical update"). */
int rg_copy_blocks(const void* src_pool, void* dst_pool, const int32_t* block_mapping,
                   int32_t num_pairs, int64_t block_bytes, int64_t src_block_stride_bytes,
                   int64_t dst_block_stride_bytes, int32_t num_layers,
                   int64_t src_layer_stride_bytes, int64_t dst_layer_stride_bytes,
                   void* stream);

/* ------------------------------------------------- model element-wise ops -- */

/* Fused residual add + RMSNorm over rows of hidden_size elements:
 *   residual != NULL: residual <- round(residual + x);  y = residual
 *   residual == NULL: y = x
 *   out = round(y / sqrt(mean(y^2) + eps) * weight), the mean and the
 *   normalisation in fp32.
 * x, residual, out: [num_rows, hidden_size]; weight: [hidden_size]; out may
 * not alias x or residual.  Replaces the candle RmsNorm and residual add
 * around each sublayer (crates/vllm-models/src/llama/architecture.rs:38-59,
 * :141-156; candle_nn::RmsNorm). */
int rg_rms_norm(const void* x, void* residual, const void* weight, void* out,
                float eps, int32_t num_rows, int32_t hidden_size, int32_t dtype,
                void* stream);

/* SwiGLU gate: out[r, i] = round(round(silu(g)) * u), g = gate_up[r, i],
 * u = gate_up[r, intermediate_size + i], silu(g) = g / (1 + exp(-g)).
 * gate_up: [num_rows, 2*intermediate_size] (the gate and up projections as
 * one GEMM), out: [num_rows, intermediate_size], num_rows <= 65535.
 * Replaces silu(gate_proj(x)) * up_proj(x) of LlamaMLP::forward
 * (crates/vllm-models/src/llama/architecture.rs:80-84). */
int rg_silu_and_mul(const void* gate_up, void* out, int32_t num_rows,
                    int32_t intermediate_size, int32_t dtype, void* stream);

/* Decode-step projection (candle's Linear::forward on a [tokens, in_features] activation,
 * crates/vllm-models/src/llama/architecture.rs:38-59,80-84, attention.rs:104-133):
 *   out[m, n] = round(sum_k x[m, k] * weight[n, k]),  m < num_rows, n < out_features,
 * bf16 / f16 operands and output, fp32 accumulation in a fixed order (deterministic).  x is
 * [num_rows, in_features], weight [out_features, in_features] (PyTorch / candle layout),
 * out [num_rows, out_features]; each with its own row stride in elements.  Shaped for decode
 * batches: num_rows <= 128, out_features a multiple of 16, in_features a positive multiple of
 * 128, x and weight rows 16-byte aligned, out rows 8-byte aligned; RG_ERR_NOT_SUPPORTED
 * otherwise (larger batches belong to a library GEMM).  A workspace of
 * rg_linear_workspace_bytes (16-byte aligned) lets narrow or deep layers split K over more
 * workgroups; without it (NULL, or smaller) the call runs unsplit.  New entry: the reference
 * runs these projections through candle's cuBLAS GEMMs. */
int rg_linear(const void* x, const void* weight, void* out, int32_t num_rows,
              int32_t out_features, int32_t in_features, int64_t x_row_stride,
              int64_t weight_row_stride, int64_t out_row_stride, void* workspace,
              size_t workspace_bytes, int32_t dtype, void* stream);

/* Bytes of the split-K workspace rg_linear uses for this shape on the current device (0: the
 * shape runs unsplit, or is not supported). */
size_t rg_linear_workspace_bytes(int32_t num_rows, int32_t out_features, int32_t in_features);

/* The gate/up projection and SiLU·mul in one pass (LlamaMLP, architecture.rs:80-84):
 *   out[m, i] = round(round(silu(g)) * u),  g = round(x[m] . gate[i]), u = round(x[m] . up[i]),
 * the arithmetic of rg_linear followed by rg_silu_and_mul.  weight_gate_up is [2 I, K] with the
 * gate and up rows interleaved in blocks of 16 (rows 32j .. 32j+15: gate rows 16j .., rows
 * 32j+16 .. 32j+31: up rows 16j ..); out is [num_rows, I].  The constraints of rg_linear, and
 * I a multiple of 16.  New entry (the reference runs two GEMMs and the element-wise product). */
int rg_linear_silu_mul(const void* x, const void* weight_gate_up, void* out, int32_t num_rows,
                       int32_t intermediate_size, int32_t in_features, int64_t x_row_stride,
                       int64_t weight_row_stride, int64_t out_row_stride, int32_t dtype, void* stream);

/* The fused q/k/v projection and rg_qkv_rope_reshape_and_cache in one pass, for decode batches
 * (the constraints of rg_linear): x [num_tokens, in_features] . weight_qkv^T, weight_qkv
 * [(H + 2 H_kv) head_dim, in_features] (q, k, v heads in that order); each head's columns are
 * rounded as the projection's output, q and k heads rotated by cos_sin[positions[t]] and
 * rounded, q written to q_out [num_tokens, H, head_dim] (q_out_token_stride elements between
 * tokens), k and v written into the paged caches at slot_mapping[t] (negative: padding, not
 * written) — the arithmetic of rg_linear followed by rg_qkv_rope_reshape_and_cache.  head_dim 32
 * or 64 (a workgroup's column tile is one head); cos_sin, the caches and kv_block_stride 16-byte
 * aligned.  New entry (the reference projects q, k and v separately and applies no RoPE,
 * attention.rs:104-125). */
int rg_linear_qkv_rope_reshape_and_cache(const void* x, const void* weight_qkv, void* q_out,
                                         void* k_cache, void* v_cache, const float* cos_sin,
                                         const int32_t* positions, const int32_t* slot_mapping,
                                         int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t block_size, int32_t in_features,
                                         int64_t x_row_stride, int64_t weight_row_stride,
                                         int64_t q_out_token_stride, int64_t kv_block_stride,
                                         int32_t dtype, void* stream);

/* A decode-step projection added to the residual stream (the o_proj / down_proj output and the
 * residual add of the next RmsNorm, architecture.rs:50-57):
 *   residual[m, n] = round(residual[m, n] + round(x[m] . weight[n])),
 * the arithmetic of rg_linear followed by the residual add of rg_rms_norm.  residual is
 * [num_rows, out_features] (residual_row_stride elements between rows) and must not overlap x or
 * weight; the constraints and the optional split-K workspace of rg_linear
 * (rg_linear_workspace_bytes).  New entry. */
int rg_linear_residual(const void* x, const void* weight, void* residual, int32_t num_rows,
                       int32_t out_features, int32_t in_features, int64_t x_row_stride,
                       int64_t weight_row_stride, int64_t residual_row_stride, void* workspace,
                       size_t workspace_bytes, int32_t dtype, void* stream);

/* RmsNorm of the residual stream folded into the projection that follows it (architecture.rs:
 * 49-50 with 104-125, and 56-57 with 80-84): with s_m = 1 / sqrt(mean_k(x[m, k]^2) + eps) over
 * the fp32 values of row m, the projection of row m is s_m * sum_k x[m, k] W[n, k] norm_weight[k]
 * with one of x[m, k] norm_weight[k] or W[n, k] norm_weight[k] rounded to the operand type, and
 * rounded as the projection's output — in place of round(x s w) . W (rg_rms_norm, then the
 * GEMM): the same values up to one rounding of each operand product.  Otherwise as
 * rg_linear_silu_mul and rg_linear_qkv_rope_reshape_and_cache; in_features at most 8192,
 * norm_weight [in_features], 16-byte aligned.  New entries. */
int rg_rms_norm_linear_silu_mul(const void* x, const void* norm_weight, float eps, const void* weight_gate_up,
                                void* out, int32_t num_rows, int32_t intermediate_size, int32_t in_features,
                                int64_t x_row_stride, int64_t weight_row_stride, int64_t out_row_stride,
                                int32_t dtype, void* stream);
int rg_rms_norm_linear_qkv_rope_reshape_and_cache(const void* x, const void* norm_weight, float eps,
                                                  const void* weight_qkv, void* q_out, void* k_cache,
                                                  void* v_cache, const float* cos_sin, const int32_t* positions,
                                                  const int32_t* slot_mapping, int32_t num_tokens,
                                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                                  int32_t block_size, int32_t in_features, int64_t x_row_stride,
                                                  int64_t weight_row_stride, int64_t q_out_token_stride,
                                                  int64_t kv_block_stride, int32_t dtype, void* stream);

/* Opt-in index checks (new entries, no counterpart: the reference's launchers pass indices to the
 * kernels unchecked, crates/vllm-cuda/src/kernels/mod.rs:196-508, as do this library's kernel
 * entries).  Each scans on the device, synchronises `stream` and returns RG_ERR_INVALID_ARGUMENT
 * naming the first bad entry, RG_OK otherwise; a debugging aid, not for graph capture.
 * rg_validate_block_tables: context_lens[s] in [0, max_blocks_per_seq * block_size] and the
 * table entries those contexts use in [0, num_blocks).  rg_validate_slot_mapping: every slot
 * below num_slots (= num_blocks * block_size; negative slots are padding). */
int rg_validate_block_tables(const int32_t* block_table, const int32_t* context_lens,
                             int32_t batch_size, int32_t max_blocks_per_seq, int32_t block_size,
                             int32_t num_blocks, void* stream);
int rg_validate_slot_mapping(const int32_t* slot_mapping, int32_t num_tokens, int64_t num_slots,
                             void* stream);

/* ------------------------------------------------------- decode, v1 -------- */

/* Bytes of workspace rg_paged_attention_v1 / _v1_plus use for the given shape on the
 * current device (0 is a valid answer: then no workspace is needed).  The workspace holds
 * split-K partials; its contents need no initialisation. */
size_t rg_paged_attention_v1_workspace_bytes(int32_t batch_size, int32_t num_heads,
                                             int32_t num_kv_heads, int32_t head_dim,
                                             int32_t block_size, int32_t max_blocks_per_seq);

/* Decode attention, one query token per sequence:
 *   out[s,h,:] = sum_t softmax_t(scale * q[s,h,:].K_t) V_t  over t < context_lens[s]
 * q/out [batch, num_heads, head_dim].  context_lens[s] == 0 gives zeros.
 * With workspace == NULL the whole context of a sequence is processed by one
 * workgroup per kv-head.  With a workspace of rg_paged_attention_v1_workspace_bytes the
 * KV blocks of the whole batch are split evenly over all compute units (each wave gets
 * the same number of blocks, whatever the context lengths) and the per-split partials are
 * merged by a second kernel — the fast path for ragged batches.  Both give the same
 * result within fp32 rounding.
 * Replaces launch_v1 (crates/vllm-cuda/src/kernels/mod.rs:305-348). */
int rg_paged_attention_v1(const void* query, const void* key_cache,
                          const void* value_cache, const int32_t* block_table,
                          const int32_t* context_lens, void* output, float scale,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t block_size, int32_t max_blocks_per_seq,
                          int32_t batch_size, int32_t dtype, int64_t kv_block_stride,
                          void* workspace, size_t workspace_bytes, void* stream);

/* One decode step's attention with its RoPE + cache pass fused in: the results of
 * rg_rope_reshape_and_cache(q', key, value, ...) on a copy q' of query, with one new
 * token per sequence (token s of key / value [batch_size, num_kv_heads, head_dim],
 * positions and slot_mapping [batch_size] belongs to sequence s), followed by
 * rg_paged_attention_v1(q', ...) — output and caches bit for bit — in the launches of
 * the stream-K decode alone.  query is read, not rotated in place.  slot_mapping[s]
 * is -1 (a padding token: nothing written) or the slot of position
 * context_lens[s] - 1 in sequence s's block table, as in every decode step; any
 * other slot is left unwritten (where the chain would write it).  Needs a workspace of
 * rg_paged_attention_v1_workspace_bytes; bf16 / f16, head_dim 64 or 128,
 * num_heads / num_kv_heads 1 to 8 (RG_ERR_NOT_SUPPORTED otherwise).
 * New entry: the reference runs RoPE, reshape_and_cache and launch_v1 as separate
 * calls (crates/vllm-cuda/src/kernels/mod.rs:196-225, 227-262, 305-348). */
int rg_rope_reshape_and_cache_paged_attention_v1(
    const void* query, const void* key, const void* value, void* key_cache,
    void* value_cache, const float* cos_sin, const int32_t* positions,
    const int32_t* slot_mapping, const int32_t* block_table,
    const int32_t* context_lens, void* output, float scale, int32_t num_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int32_t max_blocks_per_seq, int32_t batch_size, int32_t dtype,
    int64_t kv_block_stride, void* workspace, size_t workspace_bytes, void* stream);

/* Same computation as rg_paged_attention_v1, with the rotation_metadata
 * argument of launch_v1_plus (crates/vllm-cuda/src/kernels/mod.rs:350-399),
 * which is ignored (identity rotation). */
int rg_paged_attention_v1_plus(const void* query, const void* key_cache,
                               const void* value_cache, const int32_t* block_table,
                               const int32_t* context_lens, void* output,
                               const float* rotation_metadata, float scale,
                               int32_t num_heads, int32_t num_kv_heads,
                               int32_t head_dim, int32_t block_size,
                               int32_t max_blocks_per_seq, int32_t batch_size,
                               int32_t dtype, int64_t kv_block_stride,
                               void* workspace, size_t workspace_bytes, void* stream);

/* Largest split-K scratch rg_paged_attention_v1_no_alloc can use: 16 MiB, a static
 * device array of the library that every device holds from the library's load until the
 * process ends.  The stream-K form needs (W + batch*num_kv_heads) * (G*head_dim + 2G) * 4
 * bytes (+ 8 per segment), W = 4 per compute unit and G = num_heads/num_kv_heads: at
 * G = 4, head_dim 128 on 256 compute units up to 7,000 (batch x kv-head) segments fit. */
#define RG_NO_ALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/* rg_paged_attention_v1 without a workspace argument and without any allocation: the
 * stream-K split runs on the library's static scratch (RG_NO_ALLOC_SCRATCH_BYTES per
 * device, its address looked up by rg_init or by the first call on a device) instead of a
 * caller's workspace; shapes outside the stream-K path take the path
 * rg_paged_attention_v1 takes with workspace == NULL, which uses no scratch.  Same results
 * as rg_paged_attention_v1 with a workspace.  Returns RG_ERR_WORKSPACE, launching
 * nothing, when the shape needs more scratch than the static array holds.  Calls no
 * hipMalloc / hipFree / memset and records nothing that allocates, so it may run under HIP
 * graph capture.  The scratch needs no clearing (every call writes what it reads), but it
 * is shared by every call on a device: calls that overlap in time on one device (different
 * streams or threads without ordering between them) race on it; calls on one stream are
 * ordered and safe.
 * No counterpart in the reference: an entry for callers that cannot allocate device
 * memory (code under graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int rg_paged_attention_v1_no_alloc(const void* query, const void* key_cache,
                                   const void* value_cache, const int32_t* block_table,
                                   const int32_t* context_lens, void* output, float scale,
                                   int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                   int32_t block_size, int32_t max_blocks_per_seq,
                                   int32_t batch_size, int32_t dtype, int64_t kv_block_stride,
                                   void* stream);

/* ------------------------------------------------- decode, v2 split-K ------ */

/* Bytes of the three fp32 scratch arrays of v2 (tmp_out, exp_sums, max_logits)
 * for a [batch, num_heads, num_partitions, head_dim] problem, laid out
 * back-to-back in that order, each 256-byte aligned. */
size_t rg_v2_workspace_bytes(int32_t batch_size, int32_t num_heads,
                             int32_t num_partitions, int32_t head_dim);

/* Partition p of sequence s covers tokens [p*P, min((p+1)*P, ctx)).  Writes
 *   tmp_out[s,h,p,:]   = sum_t exp(x_t - m_p) V_t      (fp32, unnormalised)
 *   exp_sums[s,h,p]    = sum_t exp(x_t - m_p)
 *   max_logits[s,h,p]  = m_p = max_t x_t,   x_t = scale * q.K_t
 * Partitions with p*P >= ctx are left untouched.  P = partition_size must be a
 * positive multiple of block_size (the reference fixes P = 256,
 * crates/vllm-cuda/src/kernels/paged_attention_utils.cuh:10).
 * Replaces launch_v2_partition (crates/vllm-cuda/src/kernels/mod.rs:401-456). */
int rg_paged_attention_v2_partition(const void* query, const void* key_cache,
                                    const void* value_cache,
                                    const int32_t* block_table,
                                    const int32_t* context_lens, float* tmp_out,
                                    float* exp_sums, float* max_logits,
                                    const float* rotation_metadata, float scale,
                                    int32_t num_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t block_size,
                                    int32_t max_blocks_per_seq,
                                    int32_t num_partitions, int32_t batch_size,
                                    int32_t partition_size, int32_t dtype,
                                    int64_t kv_block_stride, void* stream);

/* Merges the ceil(ctx/P) partitions of each (s,h):
 *   M = max_p m_p, r_p = exp(m_p - M), out = sum_p r_p tmp_out_p / sum_p r_p l_p
 * ctx == 0 writes zeros.  No cap on the number of partitions (the reference
 * caps at 512, crates/vllm-cuda/src/kernels/paged_attention_v2_reduce.cu:48).
 * Replaces launch_v2_reduce (crates/vllm-cuda/src/kernels/mod.rs:458-508). */
int rg_paged_attention_v2_reduce(void* output, const float* exp_sums,
                                 const float* max_logits, const float* tmp_out,
                                 const int32_t* context_lens,
                                 const float* rotation_metadata, int32_t num_heads,
                                 int32_t head_dim, int32_t num_partitions,
                                 int32_t batch_size, int32_t partition_size,
                                 int32_t dtype, void* stream);

/* The v2 computation in one call: split-K partials merged with the exp-sum/max-logit
 * rule of v2_reduce.  With a workspace of at least
 * max(rg_v2_workspace_bytes(B,H,ceil(max_context_len/P),D), rg_paged_attention_v1_workspace_bytes)
 * bytes the splits are balanced across the compute units (as in v1); with at least
 * rg_v2_workspace_bytes it runs v2_partition + v2_reduce with partition size P.
 * The host side of PagedAttentionOp::execute's v2 branch
 * (crates/vllm-cuda/src/kernels/paged_attn_op.rs:108-158). */
int rg_paged_attention_v2(const void* query, const void* key_cache,
                          const void* value_cache, const int32_t* block_table,
                          const int32_t* context_lens, void* output, float scale,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                          int32_t block_size, int32_t max_blocks_per_seq,
                          int32_t batch_size, int32_t max_context_len,
                          int32_t partition_size, int32_t dtype,
                          int64_t kv_block_stride, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ------------------------------------------------------ packed prefill ---- */

/* Causal attention for a packed stream of new tokens (continuous batching).
 * Sequence s owns query rows [cu_seqlens[s], cu_seqlens[s+1]) of
 * query/output [num_tokens, num_heads, head_dim]; its context (prior cache +
 * these rows) has length context_lens[s] and must already be in the paged
 * cache (written by rg_reshape_and_cache / rg_rope_reshape_and_cache).
 * Row j of sequence s sits at position context_lens[s] - L_s + j and attends
 * to cache positions 0..that position inclusive, read through block_table.
 * The reference has no such kernel (it routes prefill through the decode op,
 * crates/vllm-models/src/llama/attention.rs:128-132). */
int rg_prefill_packed(const void* query, const void* key_cache,
                      const void* value_cache, const int32_t* block_table,
                      const int32_t* context_lens, const int32_t* cu_seqlens,
                      void* output, float scale, int32_t num_heads,
                      int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                      int32_t max_blocks_per_seq, int32_t num_seqs,
                      int32_t num_tokens, int32_t max_query_len, int32_t dtype,
                      int64_t kv_block_stride, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* RAILGUN_HIP_H */
