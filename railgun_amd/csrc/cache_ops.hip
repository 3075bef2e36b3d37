// KV-cache scatter (reshape_and_cache), identity-IsoQuant metadata, RoPE and the
// fused RoPE + scatter pass over the new tokens.
//
// All four are HBM-bound byte movers with no LDS.  The scatter runs one workgroup per new
// token with 16-byte vector moves along the contiguous head_dim rows wherever the row length
// and the pointers allow it; the RoPE kernels run one wave per (token, head row) so that a
// decode step's few tokens still spread over thousands of waves.
#include <algorithm>

#include <initializer_list>

#include "rg_common.hpp"

namespace rg {
namespace {

constexpr int kCacheThreads = 256;

struct CacheGeom {
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t block_size;
  int64_t kv_block_stride;  // elements
};

// Element offset of (block, kv-head, in-block offset) row in a paged cache
// (crates/vllm-cuda/src/kernels/paged_attention.cu:130-134, with an explicit
// block stride).
__device__ __forceinline__ int64_t cache_row(const CacheGeom& g, int64_t blk, int h, int off) {
  return blk * g.kv_block_stride + ((int64_t)h * g.block_size + off) * g.head_dim;
}

// One token per workgroup; copies its num_kv_heads rows of k and v with
// 16-byte (uint4) moves.  Requires head_dim*elem_bytes % 16 == 0 and 16-byte
// aligned bases / block stride (checked on the host).
__global__ __launch_bounds__(kCacheThreads) void scatter_kv_vec16(
    const uint4* __restrict__ k, const uint4* __restrict__ v, uint4* __restrict__ k_cache,
    uint4* __restrict__ v_cache, const int32_t* __restrict__ slot_mapping, CacheGeom g,
    int row_vecs, int64_t stride_vecs, float* __restrict__ rotation_metadata) {
  const int t = blockIdx.x;
  const int32_t slot = slot_mapping[t];
  if (slot < 0) return;  // padding token (paged_attention.cu:127-128)
  const int64_t blk = slot / g.block_size;
  const int off = slot % g.block_size;
  const int per_tensor = g.num_kv_heads * row_vecs;
  const int64_t src_base = (int64_t)t * per_tensor;
  for (int i = threadIdx.x; i < 2 * per_tensor; i += kCacheThreads) {
    const bool is_v = i >= per_tensor;
    const int j = is_v ? i - per_tensor : i;
    const int h = j / row_vecs;
    const int c = j - h * row_vecs;
    const int64_t dst = blk * stride_vecs + ((int64_t)h * g.block_size + off) * row_vecs + c;
    if (is_v) {
      v_cache[dst] = v[src_base + j];
    } else {
      k_cache[dst] = k[src_base + j];
    }
  }
  if (rotation_metadata != nullptr && off == 0) {
    // Identity (qL, qR) = ((0,0,0,1), (0,0,0,1)) for every 4-d group
    // (paged_attention.cu:168-173 with isoquant_utils.cuh:54-58).
    const int groups = g.num_kv_heads * (g.head_dim / 4);
    float4* meta = reinterpret_cast<float4*>(rotation_metadata) + blk * groups * 2;
    for (int i = threadIdx.x; i < groups * 2; i += kCacheThreads) {
      meta[i] = make_float4(0.f, 0.f, 0.f, 1.f);
    }
  }
}

// Element-wise fallback for rows that are not 16-byte multiples or unaligned
// pointers.  S is the storage type (float or uint16_t).
template <typename S>
__global__ __launch_bounds__(kCacheThreads) void scatter_kv_elem(
    const S* __restrict__ k, const S* __restrict__ v, S* __restrict__ k_cache,
    S* __restrict__ v_cache, const int32_t* __restrict__ slot_mapping, CacheGeom g,
    float* __restrict__ rotation_metadata) {
  const int t = blockIdx.x;
  const int32_t slot = slot_mapping[t];
  if (slot < 0) return;
  const int64_t blk = slot / g.block_size;
  const int off = slot % g.block_size;
  const int per_tensor = g.num_kv_heads * g.head_dim;
  const int64_t src_base = (int64_t)t * per_tensor;
  for (int i = threadIdx.x; i < 2 * per_tensor; i += kCacheThreads) {
    const bool is_v = i >= per_tensor;
    const int j = is_v ? i - per_tensor : i;
    const int h = j / g.head_dim;
    const int d = j - h * g.head_dim;
    const int64_t dst = cache_row(g, blk, h, off) + d;
    if (is_v) {
      v_cache[dst] = v[src_base + j];
    } else {
      k_cache[dst] = k[src_base + j];
    }
  }
  if (rotation_metadata != nullptr && off == 0) {
    const int groups = g.num_kv_heads * (g.head_dim / 4);
    float* meta = rotation_metadata + blk * groups * 8;
    for (int i = threadIdx.x; i < groups * 8; i += kCacheThreads) {
      meta[i] = ((i & 3) == 3) ? 1.f : 0.f;
    }
  }
}

// ------------------------------------------------------------------ RoPE ----

// One wave per (token, head row); each lane rotates the pairs (i, i + D/2) for
// i = lane, lane + 64, ...  `src` and `dst` are the row's element offsets (may alias).
template <typename T>
__device__ __forceinline__ void rope_row(const typename elem<T>::storage* __restrict__ src,
                                         typename elem<T>::storage* dst, const float* __restrict__ cs,
                                         int head_dim, int lane) {
  using E = elem<T>;
  const int half = head_dim / 2;
  for (int i = lane; i < half; i += 64) {
    const float lo = E::to_f32(src[i]);
    const float hi = E::to_f32(src[half + i]);
    float ol, oh;
    rope_rotate_pair(lo, hi, cs[i], cs[half + i], ol, oh);
    dst[i] = E::from_f32(ol);
    dst[half + i] = E::from_f32(oh);
  }
}

constexpr int kRowsPerGroup = kCacheThreads / 64;

// 16-byte form of rope_row for 2-byte elements: this thread rotates the pairs (i, i + D/2) for
// i in [8c, 8c + 8) with one 16-byte load and store per half and four of cos / sin.  Same
// arithmetic as rope_row (bit-identical results).
template <typename T>
__device__ __forceinline__ void rope_chunk16(const uint16_t* __restrict__ src, uint16_t* dst,
                                             const float* __restrict__ cs, int half, int c) {
  using E = elem<T>;
  const uint4 lo = *reinterpret_cast<const uint4*>(src + 8 * c);
  const uint4 hi = *reinterpret_cast<const uint4*>(src + half + 8 * c);
  const float4 c0 = *reinterpret_cast<const float4*>(cs + 8 * c);
  const float4 c1 = *reinterpret_cast<const float4*>(cs + 8 * c + 4);
  const float4 s0 = *reinterpret_cast<const float4*>(cs + half + 8 * c);
  const float4 s1 = *reinterpret_cast<const float4*>(cs + half + 8 * c + 4);
  const uint32_t lw[4] = {lo.x, lo.y, lo.z, lo.w}, hw[4] = {hi.x, hi.y, hi.z, hi.w};
  const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  uint32_t ol[4], oh[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float a0, b0, a1, b1;
    rope_rotate_pair(E::to_f32((uint16_t)(lw[k] & 0xffffu)), E::to_f32((uint16_t)(hw[k] & 0xffffu)), cv[2 * k],
                sv[2 * k], a0, b0);
    rope_rotate_pair(E::to_f32((uint16_t)(lw[k] >> 16)), E::to_f32((uint16_t)(hw[k] >> 16)), cv[2 * k + 1],
                sv[2 * k + 1], a1, b1);
    ol[k] = (uint32_t)E::from_f32(a0) | ((uint32_t)E::from_f32(a1) << 16);
    oh[k] = (uint32_t)E::from_f32(b0) | ((uint32_t)E::from_f32(b1) << 16);
  }
  *reinterpret_cast<uint4*>(dst + 8 * c) = make_uint4(ol[0], ol[1], ol[2], ol[3]);
  *reinterpret_cast<uint4*>(dst + half + 8 * c) = make_uint4(oh[0], oh[1], oh[2], oh[3]);
}

// In-place RoPE (rope.cu:11-42 semantics); grid (tokens, ceil(heads / 4)), wave = one row.
template <typename T>
__global__ __launch_bounds__(kCacheThreads) void rope_inplace_kernel(
    typename elem<T>::storage* __restrict__ x, const float* __restrict__ cos_sin,
    const int32_t* __restrict__ positions, int num_heads, int head_dim) {
  const int t = blockIdx.x;
  const int h = blockIdx.y * kRowsPerGroup + (threadIdx.x >> 6);
  if (h >= num_heads) return;
  const int64_t pos = positions[t];
  auto* row = x + ((int64_t)t * num_heads + h) * head_dim;
  rope_row<T>(row, row, cos_sin + pos * head_dim, head_dim, threadIdx.x & 63);
}

// Where the fused pass finds each token's rows: q rows are read from q_src and written,
// rotated, to q_dst (the same place for the in-place entry); k and v rows are read from
// k_src / v_src.  Strides are elements between consecutive tokens, so the q, k and v column
// ranges of one fused QKV projection output [T, (H + 2 H_kv) D] are read where they lie.
template <typename S>
struct RopeRows {
  const S* q_src;
  S* q_dst;
  const S* k_src;
  const S* v_src;
  int64_t q_src_stride, q_dst_stride, k_src_stride, v_src_stride;
};

// Fused pass over the new tokens; grid (tokens, ceil((H + 2*H_kv) / 4)), wave = one row:
// rows [0, H) rotate q, rows [H, H + H_kv) rotate k into the cache, rows
// [H + H_kv, H + 2*H_kv) copy v into the cache.
template <typename T>
__global__ __launch_bounds__(kCacheThreads) void rope_cache_kernel(
    RopeRows<typename elem<T>::storage> io, typename elem<T>::storage* __restrict__ k_cache,
    typename elem<T>::storage* __restrict__ v_cache, const float* __restrict__ cos_sin,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ slot_mapping,
    int num_heads, CacheGeom g) {
  using S = typename elem<T>::storage;
  const int t = blockIdx.x;
  const int r = blockIdx.y * kRowsPerGroup + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int D = g.head_dim;
  const int hkv = g.num_kv_heads;
  if (r >= num_heads + 2 * hkv) return;
  if (r < num_heads) {
    const int64_t pos = positions[t];
    rope_row<T>(io.q_src + t * io.q_src_stride + (int64_t)r * D, io.q_dst + t * io.q_dst_stride + (int64_t)r * D,
                cos_sin + pos * D, D, lane);
    return;
  }
  const int32_t slot = slot_mapping[t];
  if (slot < 0) return;  // padding token (paged_attention.cu:127-128)
  const int64_t blk = slot / g.block_size;
  const int off = slot % g.block_size;
  if (r < num_heads + hkv) {
    const int h = r - num_heads;
    const int64_t pos = positions[t];
    rope_row<T>(io.k_src + t * io.k_src_stride + (int64_t)h * D, k_cache + cache_row(g, blk, h, off),
                cos_sin + pos * D, D, lane);
  } else {
    const int h = r - num_heads - hkv;
    const S* src = io.v_src + t * io.v_src_stride + (int64_t)h * D;
    S* dst = v_cache + cache_row(g, blk, h, off);
    for (int i = lane; i < D; i += 64) dst[i] = src[i];
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 16-byte form of rope_cache_kernel for 2-byte elements with head_dim D a multiple of 16
// (D / 16 divides the workgroup): D / 16 threads per row (8 pairs each), so a workgroup covers
// kCacheThreads * 16 / D rows of one token; grid (tokens, row groups).  Rows, strides, the
// cache block stride and cos_sin are 16-byte aligned (checked on the host).
template <typename T>
__global__ __launch_bounds__(kCacheThreads) void rope_cache_vec_kernel(RopeRows<uint16_t> io,
                                                                       uint16_t* __restrict__ k_cache,
                                                                       uint16_t* __restrict__ v_cache,
                                                                       const float* __restrict__ cos_sin,
                                                                       const int32_t* __restrict__ positions,
                                                                       const int32_t* __restrict__ slot_mapping,
                                                                       int num_heads, CacheGeom g) {
  const int D = g.head_dim;
  const int per_row = D / 16;
  const int t = blockIdx.x;
  const int r = blockIdx.y * (kCacheThreads / per_row) + threadIdx.x / per_row;
  const int c = threadIdx.x % per_row;
  const int hkv = g.num_kv_heads;
  const int half = D / 2;
  if (r >= num_heads + 2 * hkv) return;
  if (r < num_heads) {
    const int64_t pos = positions[t];
    rope_chunk16<T>(io.q_src + t * io.q_src_stride + (int64_t)r * D, io.q_dst + t * io.q_dst_stride + (int64_t)r * D,
                    cos_sin + pos * D, half, c);
    return;
  }
  const int32_t slot = slot_mapping[t];
  if (slot < 0) return;  // padding token (paged_attention.cu:127-128)
  const int64_t blk = slot / g.block_size;
  const int off = slot % g.block_size;
  if (r < num_heads + hkv) {
    const int h = r - num_heads;
    const int64_t pos = positions[t];
    rope_chunk16<T>(io.k_src + t * io.k_src_stride + (int64_t)h * D, k_cache + cache_row(g, blk, h, off),
                    cos_sin + pos * D, half, c);
  } else {
    const int h = r - num_heads - hkv;
    const uint16_t* src = io.v_src + t * io.v_src_stride + (int64_t)h * D;
    uint16_t* dst = v_cache + cache_row(g, blk, h, off);
    *reinterpret_cast<uint4*>(dst + 8 * c) = *reinterpret_cast<const uint4*>(src + 8 * c);
    *reinterpret_cast<uint4*>(dst + half + 8 * c) = *reinterpret_cast<const uint4*>(src + half + 8 * c);
  }
}

// 16-byte form of rope_inplace_kernel (same conditions); grid (tokens, row groups).
template <typename T>
__global__ __launch_bounds__(kCacheThreads) void rope_inplace_vec_kernel(uint16_t* __restrict__ x,
                                                                         const float* __restrict__ cos_sin,
                                                                         const int32_t* __restrict__ positions,
                                                                         int num_heads, int head_dim) {
  const int per_row = head_dim / 16;
  const int t = blockIdx.x;
  const int h = blockIdx.y * (kCacheThreads / per_row) + threadIdx.x / per_row;
  if (h >= num_heads) return;
  const int64_t pos = positions[t];
  uint16_t* row = x + ((int64_t)t * num_heads + h) * head_dim;
  rope_chunk16<T>(row, row, cos_sin + pos * head_dim, head_dim / 2, threadIdx.x % per_row);
}

// Whether the 16-byte RoPE kernels apply (2-byte elements): head_dim a multiple of 16 whose
// 16-element chunks divide the workgroup, 16-byte aligned pointers and strides.
bool rope_vec_ok(int d, std::initializer_list<const void*> ptrs, std::initializer_list<int64_t> strides) {
  if (d % 16 != 0 || kCacheThreads % (d / 16) != 0) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  for (int64_t st : strides)
    if (st % 8 != 0) return false;
  return true;
}

// ---------------------------------------------------------------- block copy ----

// Whole-block copies between two pools: grid (pairs, layers, slices).  Pair i copies block
// mapping[2i] of the source to block mapping[2i+1] of the destination in every layer; a
// block's bytes are split into `slices` ranges so that large blocks spread over several
// workgroups.  16-byte moves (sizes and strides checked to be multiples of 16 on the host).
__global__ __launch_bounds__(kCacheThreads) void copy_blocks_kernel(const uint4* __restrict__ src,
                                                                    uint4* __restrict__ dst,
                                                                    const int32_t* __restrict__ mapping,
                                                                    int64_t block_vecs, int64_t src_block_vecs,
                                                                    int64_t dst_block_vecs, int64_t src_layer_vecs,
                                                                    int64_t dst_layer_vecs, int64_t slice_vecs) {
  const int64_t pair = blockIdx.x;
  const int64_t layer = blockIdx.y;
  const int64_t b0 = (int64_t)blockIdx.z * slice_vecs;
  const int64_t b1 = min(b0 + slice_vecs, block_vecs);
  const int64_t sb = mapping[2 * pair], db = mapping[2 * pair + 1];
  const uint4* s = src + layer * src_layer_vecs + sb * src_block_vecs;
  uint4* d = dst + layer * dst_layer_vecs + db * dst_block_vecs;
  for (int64_t i = b0 + threadIdx.x; i < b1; i += kCacheThreads) d[i] = s[i];
}

// ------------------------------------------------------------ host side ----

int check_cache_args(const char* op, const void* k, const void* v, const void* kc,
                     const void* vc, const int32_t* slots, int32_t hkv, int32_t d, int32_t bs,
                     int32_t n, int32_t dtype, int64_t stride) {
  if (dtype_bytes(dtype) == 0) return fail(RG_ERR_NOT_SUPPORTED, "%s: unknown dtype %d", op, dtype);
  if (n < 0 || hkv <= 0 || d <= 0 || bs <= 0) {
    return fail(RG_ERR_INVALID_ARGUMENT,
                "%s: need num_tokens >= 0 and positive num_kv_heads/head_dim/block_size "
                "(got %d, %d, %d, %d)", op, n, hkv, d, bs);
  }
  if (stride != 0 && stride < (int64_t)hkv * bs * d) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: kv_block_stride %lld smaller than a block (%lld)",
                op, (long long)stride, (long long)hkv * bs * d);
  }
  if (n > 0 && (!k || !v || !kc || !vc || !slots)) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  return RG_OK;
}

int launch_scatter(const char* op, const void* k, const void* v, void* k_cache, void* v_cache,
                   const int32_t* slot_mapping, float* meta, int32_t hkv, int32_t d, int32_t bs,
                   int32_t n, int32_t dtype, int64_t stride, void* stream) {
  int st = check_cache_args(op, k, v, k_cache, v_cache, slot_mapping, hkv, d, bs, n, dtype, stride);
  if (st != RG_OK) return st;
  if (meta != nullptr && d % 4 != 0) {
    return fail(RG_ERR_NOT_SUPPORTED, "%s: head_dim must be a multiple of 4, got %d", op, d);
  }
  if (n == 0) return ok();
  const int64_t stride_el = stride ? stride : (int64_t)hkv * bs * d;
  CacheGeom g{hkv, d, bs, stride_el};
  const int eb = dtype_bytes(dtype);
  const int64_t row_bytes = (int64_t)d * eb;
  hipStream_t s = as_stream(stream);
  if (row_bytes % 16 == 0 && (stride_el * eb) % 16 == 0 && aligned16(k) && aligned16(v) &&
      aligned16(k_cache) && aligned16(v_cache)) {
    const int row_vecs = (int)(row_bytes / 16);
    hipLaunchKernelGGL(scatter_kv_vec16, dim3(n), dim3(kCacheThreads), 0, s,
                       static_cast<const uint4*>(k), static_cast<const uint4*>(v),
                       static_cast<uint4*>(k_cache), static_cast<uint4*>(v_cache), slot_mapping,
                       g, row_vecs, stride_el * eb / 16, meta);
  } else if (eb == 4) {
    hipLaunchKernelGGL(scatter_kv_elem<float>, dim3(n), dim3(kCacheThreads), 0, s,
                       static_cast<const float*>(k), static_cast<const float*>(v),
                       static_cast<float*>(k_cache), static_cast<float*>(v_cache), slot_mapping,
                       g, meta);
  } else {
    hipLaunchKernelGGL(scatter_kv_elem<uint16_t>, dim3(n), dim3(kCacheThreads), 0, s,
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                       static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                       slot_mapping, g, meta);
  }
  return check_launch(op);
}

template <typename T>
int launch_rope_inplace(void* x, const float* cs, const int32_t* pos, int h, int d, int n, hipStream_t s) {
  using S = typename elem<T>::storage;
  if constexpr (sizeof(S) == 2) {
    if (rope_vec_ok(d, {x, cs}, {(int64_t)d})) {
      const int rows = kCacheThreads / (d / 16);
      hipLaunchKernelGGL(rope_inplace_vec_kernel<T>, dim3(n, (h + rows - 1) / rows), dim3(kCacheThreads), 0, s,
                         static_cast<uint16_t*>(x), cs, pos, h, d);
      return check_launch("rope");
    }
  }
  const dim3 grid(n, (h + kRowsPerGroup - 1) / kRowsPerGroup);
  hipLaunchKernelGGL(rope_inplace_kernel<T>, grid, dim3(kCacheThreads), 0, s, static_cast<S*>(x), cs, pos, h,
                     d);
  return check_launch("rope");
}

template <typename T>
int launch_rope_cache(const RopeRows<typename elem<T>::storage>& io, void* kc, void* vc, const float* cs,
                      const int32_t* pos, const int32_t* slots, int h, CacheGeom g, int n, hipStream_t s,
                      const char* op) {
  using S = typename elem<T>::storage;
  const int rows = h + 2 * g.num_kv_heads;
  if constexpr (sizeof(S) == 2) {
    if (rope_vec_ok(g.head_dim, {io.q_src, io.q_dst, io.k_src, io.v_src, kc, vc, cs},
                    {io.q_src_stride, io.q_dst_stride, io.k_src_stride, io.v_src_stride, g.kv_block_stride})) {
      const int per_wg = kCacheThreads / (g.head_dim / 16);
      hipLaunchKernelGGL(rope_cache_vec_kernel<T>, dim3(n, (rows + per_wg - 1) / per_wg), dim3(kCacheThreads), 0, s,
                         io, static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc), cs, pos, slots, h, g);
      return check_launch(op);
    }
  }
  const dim3 grid(n, (rows + kRowsPerGroup - 1) / kRowsPerGroup);
  hipLaunchKernelGGL(rope_cache_kernel<T>, grid, dim3(kCacheThreads), 0, s, io, static_cast<S*>(kc),
                     static_cast<S*>(vc), cs, pos, slots, h, g);
  return check_launch(op);
}

// Argument checks shared by the two fused entries.
int check_rope_cache_args(const char* op, const void* q, const void* k, const void* v, const void* kc,
                          const void* vc, const float* cs, const int32_t* pos, const int32_t* slots, int32_t h,
                          int32_t hkv, int32_t d, int32_t bs, int32_t n, int32_t dtype, int64_t stride) {
  int st = check_cache_args(op, k, v, kc, vc, slots, hkv, d, bs, n, dtype, stride);
  if (st != RG_OK) return st;
  if (h <= 0 || d % 2 != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: need num_heads > 0 and an even head_dim", op);
  }
  if (h % hkv != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: num_heads %d not a multiple of num_kv_heads %d", op, h, hkv);
  }
  if (n > 0 && (!q || !cs || !pos)) return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer", op);
  return RG_OK;
}

}  // namespace

int probe_cache_kernels() {
  hipFuncAttributes a;
  if (hipFuncGetAttributes(&a, reinterpret_cast<const void*>(scatter_kv_vec16)) != hipSuccess ||
      hipFuncGetAttributes(&a, reinterpret_cast<const void*>(rope_cache_kernel<bf16_t>)) !=
          hipSuccess) {
    return fail(RG_ERR_HIP, "failed to load the KV-cache kernels: %s",
                hipGetErrorString(hipGetLastError()));
  }
  return RG_OK;
}

}  // namespace rg

using namespace rg;

extern "C" int rg_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                                    const int32_t* slot_mapping, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t block_size, int32_t num_tokens,
                                    int32_t dtype, int64_t kv_block_stride, void* stream) {
  return launch_scatter("reshape_and_cache", k, v, k_cache, v_cache, slot_mapping, nullptr,
                        num_kv_heads, head_dim, block_size, num_tokens, dtype, kv_block_stride,
                        stream);
}

extern "C" int rg_reshape_and_cache_isoquant(const void* k, const void* v, void* k_cache,
                                             void* v_cache, const int32_t* slot_mapping,
                                             float* rotation_metadata, int32_t num_kv_heads,
                                             int32_t head_dim, int32_t block_size,
                                             int32_t num_tokens, int32_t dtype,
                                             int64_t kv_block_stride, void* stream) {
  if (rotation_metadata == nullptr && num_tokens > 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "reshape_and_cache_isoquant: null rotation_metadata");
  }
  return launch_scatter("reshape_and_cache_isoquant", k, v, k_cache, v_cache, slot_mapping,
                        rotation_metadata, num_kv_heads, head_dim, block_size, num_tokens, dtype,
                        kv_block_stride, stream);
}

extern "C" int rg_rope(void* x, const float* cos_sin, const int32_t* positions, int32_t num_heads,
                       int32_t head_dim, int32_t num_tokens, int32_t dtype, void* stream) {
  if (dtype_bytes(dtype) == 0) return fail(RG_ERR_NOT_SUPPORTED, "rope: unknown dtype %d", dtype);
  if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT,
                "rope: need num_tokens >= 0, num_heads > 0 and an even head_dim > 0 "
                "(got %d, %d, %d)", num_tokens, num_heads, head_dim);
  }
  if (num_tokens == 0) return ok();
  if (!x || !cos_sin || !positions) return fail(RG_ERR_INVALID_ARGUMENT, "rope: null pointer");
  hipStream_t s = as_stream(stream);
  return dispatch_dtype(dtype, [&](auto tag) {
    return launch_rope_inplace<decltype(tag)>(x, cos_sin, positions, num_heads, head_dim,
                                              num_tokens, s);
  });
}

extern "C" int rg_rope_reshape_and_cache(void* q, const void* k, const void* v, void* k_cache,
                                         void* v_cache, const float* cos_sin,
                                         const int32_t* positions, const int32_t* slot_mapping,
                                         int32_t num_heads, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t block_size,
                                         int32_t num_tokens, int32_t dtype,
                                         int64_t kv_block_stride, void* stream) {
  const char* op = "rope_reshape_and_cache";
  int st = check_rope_cache_args(op, q, k, v, k_cache, v_cache, cos_sin, positions, slot_mapping, num_heads,
                                 num_kv_heads, head_dim, block_size, num_tokens, dtype, kv_block_stride);
  if (st != RG_OK || num_tokens == 0) return st == RG_OK ? ok() : st;
  CacheGeom g{num_kv_heads, head_dim, block_size,
              kv_block_stride ? kv_block_stride : (int64_t)num_kv_heads * block_size * head_dim};
  hipStream_t s = as_stream(stream);
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    using S = typename elem<T>::storage;
    const int64_t qs = (int64_t)num_heads * head_dim, kvs = (int64_t)num_kv_heads * head_dim;
    const RopeRows<S> io{static_cast<const S*>(q), static_cast<S*>(q), static_cast<const S*>(k),
                         static_cast<const S*>(v), qs, qs, kvs, kvs};
    return launch_rope_cache<T>(io, k_cache, v_cache, cos_sin, positions, slot_mapping, num_heads, g, num_tokens,
                                s, op);
  });
}

extern "C" int rg_qkv_rope_reshape_and_cache(const void* qkv, int64_t qkv_token_stride, void* q_out,
                                             void* k_cache, void* v_cache, const float* cos_sin,
                                             const int32_t* positions, const int32_t* slot_mapping,
                                             int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                             int32_t block_size, int32_t num_tokens, int32_t dtype,
                                             int64_t kv_block_stride, void* stream) {
  const char* op = "qkv_rope_reshape_and_cache";
  const int64_t row = (int64_t)(num_heads + 2 * num_kv_heads) * head_dim;
  int st = check_rope_cache_args(op, q_out, qkv, qkv, k_cache, v_cache, cos_sin, positions, slot_mapping,
                                 num_heads, num_kv_heads, head_dim, block_size, num_tokens, dtype,
                                 kv_block_stride);
  if (st != RG_OK) return st;
  if (qkv_token_stride < row) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: qkv_token_stride %lld shorter than a token's q, k and v (%lld)",
                op, (long long)qkv_token_stride, (long long)row);
  }
  if (num_tokens == 0) return ok();
  CacheGeom g{num_kv_heads, head_dim, block_size,
              kv_block_stride ? kv_block_stride : (int64_t)num_kv_heads * block_size * head_dim};
  hipStream_t s = as_stream(stream);
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    using S = typename elem<T>::storage;
    const S* base = static_cast<const S*>(qkv);
    const int64_t qd = (int64_t)num_heads * head_dim, kd = (int64_t)num_kv_heads * head_dim;
    const RopeRows<S> io{base, static_cast<S*>(q_out), base + qd, base + qd + kd, qkv_token_stride, qd,
                         qkv_token_stride, qkv_token_stride};
    return launch_rope_cache<T>(io, k_cache, v_cache, cos_sin, positions, slot_mapping, num_heads, g, num_tokens,
                                s, op);
  });
}

extern "C" int rg_copy_blocks(const void* src_pool, void* dst_pool, const int32_t* block_mapping,
                              int32_t num_pairs, int64_t block_bytes, int64_t src_block_stride_bytes,
                              int64_t dst_block_stride_bytes, int32_t num_layers, int64_t src_layer_stride_bytes,
                              int64_t dst_layer_stride_bytes, void* stream) {
  const char* op = "copy_blocks";
  if (num_pairs < 0 || num_layers < 0 || block_bytes < 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: negative num_pairs, num_layers or block_bytes", op);
  }
  if (num_pairs == 0 || num_layers == 0 || block_bytes == 0) return ok();
  if (!src_pool || !dst_pool || !block_mapping) return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer", op);
  if (src_block_stride_bytes < block_bytes || dst_block_stride_bytes < block_bytes) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: block stride smaller than block_bytes", op);
  }
  if (num_layers > 1 && (src_layer_stride_bytes <= 0 || dst_layer_stride_bytes <= 0)) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: layer strides must be positive with num_layers > 1", op);
  }
  if (num_layers > 65535) return fail(RG_ERR_INVALID_ARGUMENT, "%s: num_layers > 65535", op);
  const int64_t all[5] = {block_bytes, src_block_stride_bytes, dst_block_stride_bytes,
                          num_layers > 1 ? src_layer_stride_bytes : 0, num_layers > 1 ? dst_layer_stride_bytes : 0};
  for (int64_t v : all) {
    if (v % 16 != 0) return fail(RG_ERR_NOT_SUPPORTED, "%s: sizes and strides must be multiples of 16 bytes", op);
  }
  if (!aligned16(src_pool) || !aligned16(dst_pool)) {
    return fail(RG_ERR_NOT_SUPPORTED, "%s: pool pointers must be 16-byte aligned", op);
  }
  // The kernel dereferences all three pointers: each must be memory HIP knows (device
  // memory, or pinned host memory mapped into the device's address space), never pageable
  // host memory.
  const void* ptrs[3] = {src_pool, dst_pool, block_mapping};
  const char* names[3] = {"src_pool", "dst_pool", "block_mapping"};
  for (int i = 0; i < 3; ++i) {
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, ptrs[i]) != hipSuccess || at.devicePointer == nullptr ||
        (at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeHost) || at.isManaged) {
      (void)hipGetLastError();
      return fail(RG_ERR_INVALID_ARGUMENT, "%s: %s is neither device memory nor pinned host memory", op, names[i]);
    }
  }
  const int64_t vecs = block_bytes / 16;
  // Slices of at least 16 KB per workgroup.
  const int64_t slice = std::max<int64_t>(1024, ceil_div(vecs, 64));
  const int64_t slices = ceil_div(vecs, slice);
  const dim3 grid((unsigned)num_pairs, (unsigned)num_layers, (unsigned)slices);
  hipLaunchKernelGGL(copy_blocks_kernel, grid, dim3(kCacheThreads), 0, as_stream(stream),
                     static_cast<const uint4*>(src_pool), static_cast<uint4*>(dst_pool), block_mapping, vecs,
                     src_block_stride_bytes / 16, dst_block_stride_bytes / 16, src_layer_stride_bytes / 16,
                     dst_layer_stride_bytes / 16, slice);
  return check_launch(op);
}
