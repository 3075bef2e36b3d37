// Packed causal prefill over a paged KV cache.
//
// Sequence s owns query rows [cu_seqlens[s], cu_seqlens[s+1]) of the packed
// stream; its context of context_lens[s] tokens (earlier chunks + these rows)
// is already in the paged cache.  Row j sits at absolute position
// pos = context_lens[s] - L_s + j and attends to cache positions 0..pos.
//
// prefill_generic_kernel: one wave per (row, q-head), any dtype / head_dim /
// block size; each lane owns 4 dims and the keys are visited in order with an
// online softmax.  The MFMA tile kernel for bf16/f16 lives next to it.
#include <math.h>

#include <algorithm>

#include "rg_common.hpp"

namespace rg {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

struct PrefillArgs {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_table;
  const int32_t* context_lens;
  const int32_t* cu_seqlens;
  void* out;
  float scale_log2;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t max_blocks;
  int32_t num_seqs;
  int32_t num_tokens;
  int64_t kv_stride;
};

// Sequence owning packed row `row`: the last s with cu_seqlens[s] <= row.
__device__ __forceinline__ int find_seq(const int32_t* cu, int num_seqs, int row) {
  int lo = 0, hi = num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= row) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <typename T>
__global__ __launch_bounds__(64) void prefill_generic_kernel(PrefillArgs a) {
  using E = elem<T>;
  using S = typename E::storage;
  const int row = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int D = a.head_dim;
  const int s = find_seq(a.cu_seqlens, a.num_seqs, row);
  const int L = a.cu_seqlens[s + 1] - a.cu_seqlens[s];
  const int j = row - a.cu_seqlens[s];
  const int ctx = min(a.context_lens[s], a.max_blocks * a.block_size);
  const int pos = ctx - L + j;  // keys 0..pos
  S* op = static_cast<S*>(a.out) + ((int64_t)row * a.num_heads + h) * D;
  const int d0 = lane * 4;
  const bool act = d0 < D;
  if (j >= L || pos < 0) {
    // Rows outside every sequence (or an inconsistent context) get zeros.
    if (act) {
#pragma unroll
      for (int u = 0; u < 4; ++u) E::store(op, d0 + u, 0.f);
    }
    return;
  }
  const int kvh = h / (a.num_heads / a.num_kv_heads);
  const S* qp = static_cast<const S*>(a.q) + ((int64_t)row * a.num_heads + h) * D;
  float qv[4] = {0.f, 0.f, 0.f, 0.f};
  if (act) {
#pragma unroll
    for (int u = 0; u < 4; ++u) qv[u] = E::load(qp, d0 + u);
  }
  const S* kc = static_cast<const S*>(a.k_cache);
  const S* vc = static_cast<const S*>(a.v_cache);
  const int32_t* bt = a.block_table + (int64_t)s * a.max_blocks;
  float m = -INFINITY, l = 0.f;
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  for (int t = 0; t <= pos; ++t) {
    const int64_t blk = bt[t / a.block_size];
    const int off = t % a.block_size;
    const int64_t base = blk * a.kv_stride + ((int64_t)kvh * a.block_size + off) * D;
    float kv[4] = {0.f, 0.f, 0.f, 0.f}, vv[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        kv[u] = E::load(kc, base + d0 + u);
        vv[u] = E::load(vc, base + d0 + u);
      }
    }
    const float x = wave_sum(qv[0] * kv[0] + qv[1] * kv[1] + qv[2] * kv[2] + qv[3] * kv[3]) *
                    a.scale_log2;
    const float m_new = fmaxf(m, x);
    const float alpha = exp2f(m - m_new);
    const float pe = exp2f(x - m_new);
    l = l * alpha + pe;
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = o[u] * alpha + pe * vv[u];
    m = m_new;
  }
  const float inv = 1.f / l;
  if (act) {
#pragma unroll
    for (int u = 0; u < 4; ++u) E::store(op, d0 + u, o[u] * inv);
  }
}

}  // namespace

int probe_prefill_kernels() {
  hipFuncAttributes at;
  if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(prefill_generic_kernel<bf16_t>)) !=
      hipSuccess) {
    return fail(RG_ERR_HIP, "failed to load the prefill kernels: %s",
                hipGetErrorString(hipGetLastError()));
  }
  return RG_OK;
}

}  // namespace rg

using namespace rg;

extern "C" int rg_prefill_packed(const void* query, const void* key_cache, const void* value_cache,
                                 const int32_t* block_table, const int32_t* context_lens,
                                 const int32_t* cu_seqlens, void* output, float scale,
                                 int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t block_size, int32_t max_blocks_per_seq,
                                 int32_t num_seqs, int32_t num_tokens, int32_t max_query_len,
                                 int32_t dtype, int64_t kv_block_stride, void* stream) {
  const char* op = "prefill_packed";
  (void)max_query_len;
  if (dtype_bytes(dtype) == 0) return fail(RG_ERR_NOT_SUPPORTED, "%s: unknown dtype %d", op, dtype);
  if (head_dim <= 0 || head_dim % 4 != 0 || head_dim > RG_MAX_HEAD_DIM) {
    return fail(RG_ERR_NOT_SUPPORTED,
                "not supported: PagedAttention - head_dim must be a multiple of 4 and <= %d, "
                "but got %d", RG_MAX_HEAD_DIM, head_dim);
  }
  if (num_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 || max_blocks_per_seq < 0 ||
      num_seqs < 0 || num_tokens < 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: negative or zero size argument", op);
  }
  if (num_heads % num_kv_heads != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: num_heads %d is not a multiple of num_kv_heads %d",
                op, num_heads, num_kv_heads);
  }
  const int64_t stride =
      kv_block_stride ? kv_block_stride : (int64_t)num_kv_heads * block_size * head_dim;
  if (stride < (int64_t)num_kv_heads * block_size * head_dim) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: kv_block_stride smaller than a block", op);
  }
  if (num_tokens == 0) return ok();
  if (num_seqs == 0) return fail(RG_ERR_INVALID_ARGUMENT, "%s: tokens without sequences", op);
  if (!query || !key_cache || !value_cache || !block_table || !context_lens || !cu_seqlens ||
      !output) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  PrefillArgs a{query, key_cache, value_cache, block_table, context_lens, cu_seqlens, output,
                scale * kLog2e, num_heads, num_kv_heads, head_dim, block_size,
                max_blocks_per_seq, num_seqs, num_tokens, stride};
  hipStream_t s = as_stream(stream);
  return dispatch_dtype(dtype, [&](auto tag) {
    hipLaunchKernelGGL(prefill_generic_kernel<decltype(tag)>, dim3(num_tokens, num_heads), dim3(64),
                       0, s, a);
    return check_launch(op);
  });
}
