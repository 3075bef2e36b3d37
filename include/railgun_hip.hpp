/*
 * railgun_hip.hpp — C++ host-side mirror of Railgun's kernel launchers and custom op,
 * over the C ABI of railgun_hip.h.  Header-only, C++17.
 *
 *  - railgun::PagedAttentionKernels mirrors PagedAttentionKernels
 *    (crates/vllm-cuda/src/kernels/mod.rs:23-509): one launch_* method per launcher with
 *    the reference's argument order and meaning, plus the dtype / kv_block_stride /
 *    workspace arguments of the C ABI.  Launches are asynchronous on the object's stream
 *    and never allocate.
 *  - railgun::PagedAttentionOp mirrors PagedAttentionOp
 *    (crates/vllm-cuda/src/kernels/paged_attn_op.rs:12-269): execute() with the
 *    v1 (max_context_len <= 4096) / v2 dispatch rule, reshape_and_cache(), apply_rope(),
 *    plus the fused rope_reshape_and_cache() and prefill_packed().
 *  - railgun::CoreError carries the variants of CoreError
 *    (crates/vllm-core/src/error.rs:21-77) that these calls produce: DeviceInit
 *    (construction), NotSupported (head_dim / dtype checks, mod.rs:42-54) and Tensor
 *    (launch failures and invalid arguments, mod.rs:222,258,477-482).
 *  - railgun::DeviceBuffer<T> is the owning device allocation the launchers borrow from,
 *    in place of cudarc's CudaSlice<T>; TensorView is the borrowed strided view the op
 *    takes in place of candle's Tensor.
 */
#ifndef RAILGUN_HIP_HPP
#define RAILGUN_HIP_HPP

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "railgun_hip.h"

namespace railgun {

enum class DType : int32_t { F32 = RG_DTYPE_F32, BF16 = RG_DTYPE_BF16, F16 = RG_DTYPE_F16 };

inline size_t dtype_size(DType d) { return d == DType::F32 ? 4 : 2; }

class CoreError : public std::runtime_error {
 public:
  enum class Kind { DeviceInit, NotSupported, Tensor, OutOfMemory };
  CoreError(Kind kind, const std::string& msg) : std::runtime_error(msg), kind_(kind) {}
  Kind kind() const { return kind_; }

 private:
  Kind kind_;
};

// Converts a C-ABI status into the CoreError variant the reference raises at that point.
inline void check(int status, const char* what) {
  if (status == RG_OK) return;
  const std::string msg = std::string(what) + ": " + rg_last_error();
  switch (status) {
    case RG_ERR_NOT_SUPPORTED:
      throw CoreError(CoreError::Kind::NotSupported, msg);
    default:  // RG_ERR_INVALID_ARGUMENT, RG_ERR_HIP, RG_ERR_WORKSPACE
      throw CoreError(CoreError::Kind::Tensor, msg);
  }
}

// Owning device allocation of `len` elements of T (move-only).
template <typename T>
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t len) : len_(len) {
    if (len == 0) return;
    if (hipMalloc(reinterpret_cast<void**>(&ptr_), len * sizeof(T)) != hipSuccess) {
      (void)hipGetLastError();
      throw CoreError(CoreError::Kind::OutOfMemory,
                      "out of memory: requested " + std::to_string(len * sizeof(T)) + " bytes");
    }
  }
  static DeviceBuffer from_host(const std::vector<T>& host) {
    DeviceBuffer b(host.size());
    b.copy_from_host(host);
    return b;
  }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept : ptr_(o.ptr_), len_(o.len_) { o.ptr_ = nullptr, o.len_ = 0; }
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      reset();
      ptr_ = o.ptr_, len_ = o.len_;
      o.ptr_ = nullptr, o.len_ = 0;
    }
    return *this;
  }
  ~DeviceBuffer() { reset(); }

  T* data() { return ptr_; }
  const T* data() const { return ptr_; }
  size_t len() const { return len_; }
  size_t bytes() const { return len_ * sizeof(T); }

  void copy_from_host(const std::vector<T>& host) {
    if (host.size() != len_) throw CoreError(CoreError::Kind::Tensor, "copy_from_host: size mismatch");
    if (len_ && hipMemcpy(ptr_, host.data(), bytes(), hipMemcpyHostToDevice) != hipSuccess)
      throw CoreError(CoreError::Kind::Tensor, "hipMemcpy host->device failed");
  }
  std::vector<T> to_host() const {
    std::vector<T> host(len_);
    if (len_ && hipMemcpy(host.data(), ptr_, bytes(), hipMemcpyDeviceToHost) != hipSuccess)
      throw CoreError(CoreError::Kind::Tensor, "hipMemcpy device->host failed");
    return host;
  }

 private:
  void reset() {
    if (ptr_) (void)hipFree(ptr_);
    ptr_ = nullptr;
    len_ = 0;
  }
  T* ptr_ = nullptr;
  size_t len_ = 0;
};

// Borrowed view of a device tensor: element type, shape and strides in elements.
struct TensorView {
  void* data = nullptr;
  DType dtype = DType::F32;
  std::vector<int64_t> shape;
  std::vector<int64_t> strides;

  // A contiguous (row-major) view.
  static TensorView contiguous(void* data, DType dtype, std::vector<int64_t> shape) {
    TensorView t{data, dtype, std::move(shape), {}};
    t.strides.assign(t.shape.size(), 1);
    for (int i = (int)t.shape.size() - 2; i >= 0; --i) t.strides[i] = t.strides[i + 1] * t.shape[i + 1];
    return t;
  }
  int64_t dim(int i) const { return shape.at(i); }
  int rank() const { return (int)shape.size(); }
};

class PagedAttentionKernels {
 public:
  // PagedAttentionKernels::new (mod.rs:57-190): checks the device; the code objects are
  // linked into the library, so nothing is loaded or cached here.
  explicit PagedAttentionKernels(int ordinal, hipStream_t stream = nullptr) : ordinal_(ordinal), stream_(stream) {
    if (rg_init(ordinal) != RG_OK) {
      throw CoreError(CoreError::Kind::DeviceInit,
                      "failed to initialise hip:" + std::to_string(ordinal) + ": " + rg_last_error());
    }
  }
  int ordinal() const { return ordinal_; }
  hipStream_t stream() const { return stream_; }
  void set_stream(hipStream_t s) { stream_ = s; }

  // mod.rs:196-225
  void launch_rope(void* x, const float* cos_sin, const int32_t* positions, int32_t num_heads, int32_t head_dim,
                   int32_t num_tokens, DType dtype = DType::F32) const {
    check(rg_rope(x, cos_sin, positions, num_heads, head_dim, num_tokens, (int32_t)dtype, stream_), "launch_rope");
  }
  // mod.rs:227-262
  void launch_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                                const int32_t* slot_mapping, int32_t num_kv_heads, int32_t head_dim,
                                int32_t block_size, int32_t batch_size, DType dtype = DType::F32,
                                int64_t kv_block_stride = 0) const {
    check(rg_reshape_and_cache(k, v, k_cache, v_cache, slot_mapping, num_kv_heads, head_dim, block_size,
                               batch_size, (int32_t)dtype, kv_block_stride, stream_),
          "launch_reshape_and_cache");
  }
  // mod.rs:264-303
  void launch_reshape_and_cache_isoquant(const void* k, const void* v, void* k_cache, void* v_cache,
                                         const int32_t* slot_mapping, float* rotation_metadata,
                                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                         int32_t batch_size, DType dtype = DType::F32,
                                         int64_t kv_block_stride = 0) const {
    check(rg_reshape_and_cache_isoquant(k, v, k_cache, v_cache, slot_mapping, rotation_metadata, num_kv_heads,
                                        head_dim, block_size, batch_size, (int32_t)dtype, kv_block_stride,
                                        stream_),
          "launch_reshape_and_cache_isoquant");
  }
  size_t v1_workspace_bytes(int32_t batch_size, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t block_size, int32_t max_blocks_per_seq) const {
    return rg_paged_attention_v1_workspace_bytes(batch_size, num_heads, num_kv_heads, head_dim, block_size,
                                                 max_blocks_per_seq);
  }
  // mod.rs:305-348 (workspace optional: the balanced split-K form of the same computation)
  void launch_v1(const void* query, const void* key_cache, const void* value_cache, const int32_t* block_table,
                 const int32_t* context_lens, void* output, float scale, int32_t num_heads, int32_t num_kv_heads,
                 int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq, int32_t batch_size,
                 DType dtype = DType::F32, int64_t kv_block_stride = 0, void* workspace = nullptr,
                 size_t workspace_bytes = 0) const {
    check(rg_paged_attention_v1(query, key_cache, value_cache, block_table, context_lens, output, scale, num_heads,
                                num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size, (int32_t)dtype,
                                kv_block_stride, workspace, workspace_bytes, stream_),
          "launch_v1");
  }
  // mod.rs:350-399
  void launch_v1_plus(const void* query, const void* key_cache, const void* value_cache, const int32_t* block_table,
                      const int32_t* context_lens, void* output, const float* rotation_metadata, float scale,
                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                      int32_t max_blocks_per_seq, int32_t batch_size, DType dtype = DType::F32,
                      int64_t kv_block_stride = 0, void* workspace = nullptr, size_t workspace_bytes = 0) const {
    check(rg_paged_attention_v1_plus(query, key_cache, value_cache, block_table, context_lens, output,
                                     rotation_metadata, scale, num_heads, num_kv_heads, head_dim, block_size,
                                     max_blocks_per_seq, batch_size, (int32_t)dtype, kv_block_stride, workspace,
                                     workspace_bytes, stream_),
          "launch_v1_plus");
  }
  size_t v2_workspace_bytes(int32_t batch_size, int32_t num_heads, int32_t num_partitions, int32_t head_dim) const {
    return rg_v2_workspace_bytes(batch_size, num_heads, num_partitions, head_dim);
  }
  // mod.rs:401-456
  void launch_v2_partition(const void* query, const void* key_cache, const void* value_cache,
                           const int32_t* block_table, const int32_t* context_lens, float* tmp_out,
                           float* exp_sums, float* max_logits, const float* rotation_metadata, float scale,
                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                           int32_t max_blocks_per_seq, int32_t num_partitions, int32_t batch_size,
                           int32_t partition_size = 256, DType dtype = DType::F32,
                           int64_t kv_block_stride = 0) const {
    check(rg_paged_attention_v2_partition(query, key_cache, value_cache, block_table, context_lens, tmp_out,
                                          exp_sums, max_logits, rotation_metadata, scale, num_heads, num_kv_heads,
                                          head_dim, block_size, max_blocks_per_seq, num_partitions, batch_size,
                                          partition_size, (int32_t)dtype, kv_block_stride, stream_),
          "launch_v2_partition");
  }
  // mod.rs:458-508
  void launch_v2_reduce(void* output, const float* exp_sums, const float* max_logits, const float* tmp_out,
                        const int32_t* context_lens, const float* rotation_metadata, int32_t num_heads,
                        int32_t head_dim, int32_t num_partitions, int32_t batch_size, int32_t partition_size = 256,
                        DType dtype = DType::F32) const {
    check(rg_paged_attention_v2_reduce(output, exp_sums, max_logits, tmp_out, context_lens, rotation_metadata,
                                       num_heads, head_dim, num_partitions, batch_size, partition_size,
                                       (int32_t)dtype, stream_),
          "launch_v2_reduce");
  }
  // v2 partition + reduce in one call, scratch carved from `workspace`.
  void launch_v2(const void* query, const void* key_cache, const void* value_cache, const int32_t* block_table,
                 const int32_t* context_lens, void* output, float scale, int32_t num_heads, int32_t num_kv_heads,
                 int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq, int32_t batch_size,
                 int32_t max_context_len, int32_t partition_size, void* workspace, size_t workspace_bytes,
                 DType dtype = DType::F32, int64_t kv_block_stride = 0) const {
    check(rg_paged_attention_v2(query, key_cache, value_cache, block_table, context_lens, output, scale, num_heads,
                                num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size,
                                max_context_len, partition_size, (int32_t)dtype, kv_block_stride, workspace,
                                workspace_bytes, stream_),
          "launch_v2");
  }
  // New entries (no reference launcher).
  void launch_rope_reshape_and_cache(void* q, const void* k, const void* v, void* k_cache, void* v_cache,
                                     const float* cos_sin, const int32_t* positions, const int32_t* slot_mapping,
                                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                     int32_t num_tokens, DType dtype = DType::F32,
                                     int64_t kv_block_stride = 0) const {
    check(rg_rope_reshape_and_cache(q, k, v, k_cache, v_cache, cos_sin, positions, slot_mapping, num_heads,
                                    num_kv_heads, head_dim, block_size, num_tokens, (int32_t)dtype,
                                    kv_block_stride, stream_),
          "launch_rope_reshape_and_cache");
  }
  // launch_rope_reshape_and_cache of one new token per sequence followed by launch_v1, in the
  // stream-K decode's launches (query is read, not rotated in place).
  void launch_rope_reshape_and_cache_v1(const void* query, const void* k, const void* v, void* k_cache,
                                        void* v_cache, const float* cos_sin, const int32_t* positions,
                                        const int32_t* slot_mapping, const int32_t* block_table,
                                        const int32_t* context_lens, void* output, float scale, int32_t num_heads,
                                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                        int32_t max_blocks_per_seq, int32_t batch_size, void* workspace,
                                        size_t workspace_bytes, DType dtype = DType::BF16,
                                        int64_t kv_block_stride = 0) const {
    check(rg_rope_reshape_and_cache_paged_attention_v1(
              query, k, v, k_cache, v_cache, cos_sin, positions, slot_mapping, block_table, context_lens, output,
              scale, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size, (int32_t)dtype,
              kv_block_stride, workspace, workspace_bytes, stream_),
          "launch_rope_reshape_and_cache_v1");
  }
  void launch_prefill_packed(const void* query, const void* key_cache, const void* value_cache,
                             const int32_t* block_table, const int32_t* context_lens, const int32_t* cu_seqlens,
                             void* output, float scale, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t block_size, int32_t max_blocks_per_seq, int32_t num_seqs, int32_t num_tokens,
                             int32_t max_query_len, DType dtype = DType::F32, int64_t kv_block_stride = 0) const {
    check(rg_prefill_packed(query, key_cache, value_cache, block_table, context_lens, cu_seqlens, output, scale,
                            num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, num_seqs,
                            num_tokens, max_query_len, (int32_t)dtype, kv_block_stride, stream_),
          "launch_prefill_packed");
  }

 private:
  int ordinal_;
  hipStream_t stream_;
};

// PagedAttentionOp (paged_attn_op.rs:12-19) over TensorViews.  execute() returns a new
// output buffer, as the reference returns a new Tensor; the split-K workspace is kept by
// the op and grown on demand instead of being allocated on every call (calls on one op
// must share its kernels' stream).
class PagedAttentionOp {
 public:
  static constexpr int32_t kV1MaxContext = 4096;   // paged_attn_op.rs:89
  static constexpr int32_t kV2PartitionSize = 512;

  PagedAttentionOp(float scale, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                   std::shared_ptr<PagedAttentionKernels> kernels)
      : scale_(scale), num_heads_(num_heads), num_kv_heads_(num_kv_heads), head_dim_(head_dim),
        block_size_(block_size), kernels_(std::move(kernels)) {}

  // paged_attn_op.rs:45-166: q [B, H, D] -> output [B, H, D] of q's dtype.
  DeviceBuffer<uint8_t> execute(const TensorView& q, const TensorView& k_cache, const TensorView& v_cache,
                                const TensorView& block_table, const TensorView& context_lens,
                                const float* rotation_metadata, int32_t max_context_len) {
    if (head_dim_ % 4 != 0) {
      throw CoreError(CoreError::Kind::NotSupported,
                      "Head dimension (" + std::to_string(head_dim_) + ") must be a multiple of 4 for IsoQuant.");
    }
    if (q.rank() != 3) throw CoreError(CoreError::Kind::Tensor, "q must be [batch, num_heads, head_dim]");
    const int32_t batch = (int32_t)q.dim(0), num_heads = (int32_t)q.dim(1), head_dim = (int32_t)q.dim(2);
    const int64_t kv_stride = cache_block_stride(k_cache, v_cache);
    const int32_t block_size = (int32_t)k_cache.dim(2);
    const int32_t max_blocks = (int32_t)block_table.dim(1);
    DeviceBuffer<uint8_t> out((size_t)batch * num_heads * head_dim * dtype_size(q.dtype));
    const auto* bt = static_cast<const int32_t*>(block_table.data);
    const auto* ctx = static_cast<const int32_t*>(context_lens.data);
    const size_t v1_ws = kernels_->v1_workspace_bytes(batch, num_heads, num_kv_heads_, head_dim, block_size,
                                                      max_blocks);
    if (max_context_len <= kV1MaxContext) {
      void* ws = reserve(v1_ws);
      kernels_->launch_v1_plus(q.data, k_cache.data, v_cache.data, bt, ctx, out.data(), rotation_metadata, scale_,
                               num_heads, num_kv_heads_, head_dim, block_size, max_blocks, batch, q.dtype,
                               kv_stride, ws, v1_ws);
    } else {
      const int32_t parts = (max_context_len + kV2PartitionSize - 1) / kV2PartitionSize;
      const size_t need = std::max(kernels_->v2_workspace_bytes(batch, num_heads, parts, head_dim), v1_ws);
      void* ws = reserve(need);
      kernels_->launch_v2(q.data, k_cache.data, v_cache.data, bt, ctx, out.data(), scale_, num_heads,
                          num_kv_heads_, head_dim, block_size, max_blocks, batch, max_context_len,
                          kV2PartitionSize, ws, need, q.dtype, kv_stride);
    }
    return out;
  }

  // paged_attn_op.rs:168-233: k, v [T, H_kv, D] into the caches (in place).
  void reshape_and_cache(const TensorView& k, const TensorView& v, const TensorView& k_cache,
                         const TensorView& v_cache, const int32_t* slot_mapping, float* rotation_metadata,
                         bool use_isoquant) {
    const int32_t tokens = (int32_t)k.dim(0), hkv = (int32_t)k.dim(1), d = (int32_t)k.dim(2);
    const int64_t kv_stride = cache_block_stride(k_cache, v_cache);
    if (use_isoquant) {
      kernels_->launch_reshape_and_cache_isoquant(k.data, v.data, k_cache.data, v_cache.data, slot_mapping,
                                                  rotation_metadata, hkv, d, block_size_, tokens, k.dtype,
                                                  kv_stride);
    } else {
      kernels_->launch_reshape_and_cache(k.data, v.data, k_cache.data, v_cache.data, slot_mapping, hkv, d,
                                         block_size_, tokens, k.dtype, kv_stride);
    }
  }

  // paged_attn_op.rs:236-268: in-place RoPE on x [T, H, D].
  void apply_rope(const TensorView& x, const float* cos_sin, const int32_t* positions) {
    kernels_->launch_rope(x.data, cos_sin, positions, (int32_t)x.dim(1), (int32_t)x.dim(2), (int32_t)x.dim(0),
                          x.dtype);
  }

  // RoPE on q (in place) and k, then the cache write, in one pass over the new tokens.
  void rope_reshape_and_cache(const TensorView& q, const TensorView& k, const TensorView& v,
                              const TensorView& k_cache, const TensorView& v_cache, const float* cos_sin,
                              const int32_t* positions, const int32_t* slot_mapping) {
    kernels_->launch_rope_reshape_and_cache(q.data, k.data, v.data, k_cache.data, v_cache.data, cos_sin, positions,
                                            slot_mapping, num_heads_, num_kv_heads_, head_dim_, block_size_,
                                            (int32_t)q.dim(0), q.dtype, cache_block_stride(k_cache, v_cache));
  }

  // Causal attention of the packed new tokens q [T, H, D] over the paged cache.
  DeviceBuffer<uint8_t> prefill_packed(const TensorView& q, const TensorView& k_cache, const TensorView& v_cache,
                                       const TensorView& block_table, const TensorView& context_lens,
                                       const TensorView& cu_seqlens, int32_t max_query_len) {
    const int32_t tokens = (int32_t)q.dim(0);
    DeviceBuffer<uint8_t> out((size_t)tokens * num_heads_ * head_dim_ * dtype_size(q.dtype));
    kernels_->launch_prefill_packed(q.data, k_cache.data, v_cache.data,
                                    static_cast<const int32_t*>(block_table.data),
                                    static_cast<const int32_t*>(context_lens.data),
                                    static_cast<const int32_t*>(cu_seqlens.data), out.data(), scale_, num_heads_,
                                    num_kv_heads_, head_dim_, block_size_, (int32_t)block_table.dim(1),
                                    (int32_t)cu_seqlens.dim(0) - 1, tokens, max_query_len, q.dtype,
                                    cache_block_stride(k_cache, v_cache));
    return out;
  }

 private:
  // Block stride of [NB, H_kv, bs, D] cache views whose blocks are contiguous; both caches
  // must share it (Railgun's fused pool views, block.rs:70,89-95, qualify).
  int64_t cache_block_stride(const TensorView& k_cache, const TensorView& v_cache) const {
    if (k_cache.rank() != 4 || v_cache.rank() != 4 || k_cache.shape != v_cache.shape)
      throw CoreError(CoreError::Kind::Tensor, "caches must be [num_blocks, num_kv_heads, block_size, head_dim]");
    const int64_t bs = k_cache.dim(2), d = k_cache.dim(3);
    for (const TensorView* c : {&k_cache, &v_cache}) {
      if (c->strides.size() != 4 || c->strides[3] != 1 || c->strides[2] != d || c->strides[1] != bs * d)
        throw CoreError(CoreError::Kind::Tensor, "cache blocks must be contiguous [H_kv, bs, D]");
    }
    if (k_cache.strides[0] != v_cache.strides[0] || k_cache.dtype != v_cache.dtype)
      throw CoreError(CoreError::Kind::Tensor, "k and v caches must share dtype and block stride");
    if (k_cache.dim(1) != num_kv_heads_)
      throw CoreError(CoreError::Kind::Tensor, "cache kv-head count differs from the op's");
    return k_cache.strides[0];
  }
  void* reserve(size_t bytes) {
    if (bytes == 0) return nullptr;
    if (workspace_.bytes() < bytes) {
      if (hipStreamSynchronize(kernels_->stream()) != hipSuccess)  // earlier calls may still use it
        throw CoreError(CoreError::Kind::Tensor, "hipStreamSynchronize failed");
      workspace_ = DeviceBuffer<uint8_t>(bytes);
    }
    return workspace_.data();
  }

  float scale_;
  int32_t num_heads_, num_kv_heads_, head_dim_, block_size_;
  std::shared_ptr<PagedAttentionKernels> kernels_;
  DeviceBuffer<uint8_t> workspace_;
};

}  // namespace railgun

#endif  // RAILGUN_HIP_HPP
