// Packed causal prefill over a paged KV cache.
//
// Sequence s owns query rows [cu_seqlens[s], cu_seqlens[s+1]) of the packed
// stream; its context of context_lens[s] tokens (earlier chunks + these rows)
// is already in the paged cache.  Row j sits at absolute position
// pos = context_lens[s] - L_s + j and attends to cache positions 0..pos.
//
// prefill_generic_kernel: one wave per (row, q-head), any dtype / head_dim /
// block size; each lane owns 4 dims and the keys are visited in order with an
// online softmax.  prefill_mfma_kernel (bf16/f16, GQA 4, head_dim 64/128) is the
// MFMA tile kernel used whenever it applies.
#include <math.h>

#include <algorithm>
#include <type_traits>

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

// ------------------------------------------------------------------ MFMA ----
//
// Tile = 32 queries of one sequence x the G = 4 q-heads of one kv-head; one wave per head.
// Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16 (K rows as the A
// operand straight from the paged cache, Q^T as the B operand held in registers), so that
// lane l owns query column l % 32 and the other half of its 32 keys sits in lane l ^ 32:
// the softmax statistics are per-lane scalars.  The probabilities leave that MFMA in the
// layout the B operand of O^T = V^T P^T needs (keys 16n+4h+r and 16n+8+4h+r in k-slots
// 8h..8h+7, h = lane/32), so P never goes through LDS; V is staged transposed in LDS
// (V^T[d][key], double buffered) by the whole workgroup, and the A-operand reads use the
// same key permutation.  Key tiles of 32 keys run from 0 to the last position of the tile;
// only the tiles that reach past the first query position are masked.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <typename T> struct mfma32;
template <> struct mfma32<bf16_t> {
  __device__ static __forceinline__ f32x16_t run(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct mfma32<f16_t> {
  __device__ static __forceinline__ f32x16_t run(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};

constexpr int kPT = 32;               // queries per tile and keys per key tile
constexpr int kPWaves = 4;            // one wave per q-head of the group (GQA 4)
constexpr int kPThreads = kPWaves * 64;
constexpr int kVtRow = kPT + 2;       // V^T row stride in elements (odd dword count: no bank conflicts)

// Tile `ti` of the longest-first order: rank r = 0 holds the last tile of every sequence,
// rank 1 the one before, ...; within a rank, sequences in order.  Returns false if `ti` is
// past the last tile.  All lanes of the wave get the same (s, t).
__device__ __forceinline__ bool tile_of(const int32_t* cu, int num_seqs, int ti, int lane, int& s_out,
                                        int& t_out) {
  int maxn = 0;
  for (int c0 = 0; c0 < num_seqs; c0 += 64) {
    const int sidx = c0 + lane;
    const int n = sidx < num_seqs ? (cu[sidx + 1] - cu[sidx] + kPT - 1) / kPT : 0;
    maxn = max(maxn, n);
  }
  maxn = (int)wave_max((float)maxn);
  int base = 0;
  for (int r = 0; r < maxn; ++r) {
    for (int c0 = 0; c0 < num_seqs; c0 += 64) {
      const int sidx = c0 + lane;
      const int n = sidx < num_seqs ? (cu[sidx + 1] - cu[sidx] + kPT - 1) / kPT : 0;
      const uint64_t has = __ballot(n > r);
      const int cnt = __popcll(has);
      if (ti < base + cnt) {
        // the (ti - base)-th set bit
        uint64_t m = has;
        for (int k = 0; k < ti - base; ++k) m &= m - 1;
        const int l = __ffsll((unsigned long long)m) - 1;
        s_out = c0 + l;
        const int nl = __shfl(n, l, 64);
        t_out = nl - 1 - r;
        return true;
      }
      base += cnt;
    }
  }
  return false;
}

template <typename T, int D>
__global__ __launch_bounds__(kPThreads) void prefill_mfma_kernel(
    PrefillArgs a, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ context_lens, const int32_t* __restrict__ cu_seqlens) {
  using MF = mfma32<T>;
  using S = uint16_t;
  constexpr int G = kPWaves;
  constexpr int NKC = D / 16;      // 16-element d chunks = QK MFMAs per key tile
  constexpr int NDB = D / 32;      // 32-row d blocks of O^T
  constexpr int VITEMS = 16 * (D / 8);  // (key pair, 8-d chunk) items of a V tile
  constexpr int VPER = (VITEMS + kPThreads - 1) / kPThreads;
  __shared__ uint32_t vt_lds[2][D * kVtRow / 2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int hkv = a.num_kv_heads;
  const int kvh = blockIdx.x % hkv;
  const int ti = blockIdx.x / hkv;
  int s, t;
  if (!tile_of(cu_seqlens, a.num_seqs, ti, lane, s, t)) return;
  s = __builtin_amdgcn_readfirstlane(s);
  t = __builtin_amdgcn_readfirstlane(t);

  const int row0 = cu_seqlens[s];
  const int L = cu_seqlens[s + 1] - row0;
  const int ctx = min(context_lens[s], a.max_blocks * a.block_size);
  const int prior = ctx - L;
  const int q0 = t * kPT;                      // first query of the tile (within the sequence)
  const int nq = min(kPT, L - q0);
  const int pos_min = prior + q0;
  const int pos_max = prior + q0 + nq - 1;
  const int head = kvh * G + w;
  const int H = a.num_heads;
  const int j = lane & 31;                     // query column owned by this lane
  const int hh = lane >> 5;                    // which half of the k-slots
  const bool q_valid = j < nq && pos_min >= 0;
  const int my_pos = pos_min + j;

  // Q^T operand (B): lane holds q[query j][16i + 8hh .. +8] for every d chunk i.
  uint4 qb[NKC];
  {
    const uint4* qr = reinterpret_cast<const uint4*>(q + ((int64_t)(row0 + q0 + (q_valid ? j : 0)) * H + head) * D);
#pragma unroll
    for (int i = 0; i < NKC; ++i) qb[i] = q_valid ? qr[2 * i + hh] : make_uint4(0, 0, 0, 0);
  }
  const int32_t* bt = block_table + (int64_t)s * a.max_blocks;
  const int bs = a.block_size;
  const int64_t head_off = (int64_t)kvh * bs * D;
  auto key_row = [&](int key) -> int64_t {
    const int b = min(key / bs, a.max_blocks - 1);
    return (int64_t)bt[b] * a.kv_stride + head_off + (int64_t)(key % bs) * D;
  };
  // K operand (A) of key tile kt: lane holds K[key 32kt + j][16i + 8hh .. +8].
  auto load_k = [&](int kt, uint4 (&kr)[NKC]) {
    const uint4* kp = reinterpret_cast<const uint4*>(kc + key_row(kt * kPT + j));
#pragma unroll
    for (int i = 0; i < NKC; ++i) kr[i] = kp[2 * i + hh];
  };
  // V rows of the tile for this thread's items: keys 2kp and 2kp+1, dims 8dc..8dc+8.
  auto load_v = [&](int kt, uint4 (&v0)[VPER], uint4 (&v1)[VPER]) {
#pragma unroll
    for (int u = 0; u < VPER; ++u) {
      const int item = tid + u * kPThreads;
      const int kp = item & 15;
      const int dc = item >> 4;
      const int key = kt * kPT + 2 * kp;
      if (item >= VITEMS) break;
      v0[u] = key <= pos_max ? *reinterpret_cast<const uint4*>(vc + key_row(key) + 8 * dc) : make_uint4(0, 0, 0, 0);
      v1[u] = key + 1 <= pos_max ? *reinterpret_cast<const uint4*>(vc + key_row(key + 1) + 8 * dc)
                                 : make_uint4(0, 0, 0, 0);
    }
  };
  // Transposed store: V^T[8dc + e][2kp .. 2kp+1] = (V[2kp][8dc+e], V[2kp+1][8dc+e]).
  auto store_vt = [&](int buf, const uint4 (&v0)[VPER], const uint4 (&v1)[VPER]) {
#pragma unroll
    for (int u = 0; u < VPER; ++u) {
      const int item = tid + u * kPThreads;
      const int kp = item & 15;
      const int dc = item >> 4;
      if (item >= VITEMS) break;
      const uint32_t a4[4] = {v0[u].x, v0[u].y, v0[u].z, v0[u].w};
      const uint32_t b4[4] = {v1[u].x, v1[u].y, v1[u].z, v1[u].w};
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const uint32_t lo = (a4[e2] & 0xffffu) | (b4[e2] << 16);
        const uint32_t hi = (a4[e2] >> 16) | (b4[e2] & 0xffff0000u);
        vt_lds[buf][((8 * dc + 2 * e2) * kVtRow) / 2 + kp] = lo;
        vt_lds[buf][((8 * dc + 2 * e2 + 1) * kVtRow) / 2 + kp] = hi;
      }
    }
  };

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const int nkt = pos_max / kPT + 1;
  uint4 kr[NKC];
  uint4 v0[VPER], v1[VPER];
  load_k(0, kr);
  load_v(0, v0, v1);
  store_vt(0, v0, v1);
  __syncthreads();

  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nkt;
    uint4 kn[NKC];
    if (more) {
      load_k(kt + 1, kn);
      load_v(kt + 1, v0, v1);
    }
    // S^T = K Q^T: c[4jb + r] is key 8jb + 4hh + r of the tile for query j.
    f32x16_t c;
#pragma unroll
    for (int v = 0; v < 16; ++v) c[v] = 0.f;
#pragma unroll
    for (int i = 0; i < NKC; ++i) c = MF::run(kr[i], qb[i], c);

    const int k0 = kt * kPT;
    const bool masked = k0 + kPT - 1 > pos_min;
    float sc[16];
    float tmax = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = k0 + 8 * (v >> 2) + 4 * hh + (v & 3);
      float x = c[v] * a.scale_log2;
      if (masked && key > my_pos) x = -INFINITY;
      sc[v] = x;
      tmax = fmaxf(tmax, x);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.f;
    uint32_t pk[8];
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      const float p0 = __builtin_amdgcn_exp2f(sc[v] - m_new);
      const float p1 = __builtin_amdgcn_exp2f(sc[v + 1] - m_new);
      psum += p0 + p1;
      pk[v / 2] = (uint32_t)elem<T>::from_f32(p0) | ((uint32_t)elem<T>::from_f32(p1) << 16);
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
    }
    // O^T += V^T P^T over the tile's keys, in two 16-key MFMA steps.
    const uint32_t* vt = vt_lds[buf];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const uint4 pb = make_uint4(pk[4 * n], pk[4 * n + 1], pk[4 * n + 2], pk[4 * n + 3]);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int d = 32 * db + j;
        const int e0 = (d * kVtRow + 16 * n + 4 * hh) / 2;   // keys 16n+4hh .. +4
        const int e1 = (d * kVtRow + 16 * n + 8 + 4 * hh) / 2;  // keys 16n+8+4hh .. +4
        const uint4 va = make_uint4(vt[e0], vt[e0 + 1], vt[e1], vt[e1 + 1]);
        o[db] = MF::run(va, pb, o[db]);
      }
    }
    if (more) {
      store_vt(buf ^ 1, v0, v1);
#pragma unroll
      for (int i = 0; i < NKC; ++i) kr[i] = kn[i];
    }
    __syncthreads();
  }

  // Normalise (the two halves of a query's keys live in lanes l and l ^ 32) and write.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (!q_valid) return;
  const float inv = 1.f / l_tot;
  S* orow = static_cast<S*>(a.out) + ((int64_t)(row0 + q0 + j) * H + head) * D;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int d0 = 32 * db + 8 * jb + 4 * hh;
      const uint32_t w0 = (uint32_t)elem<T>::from_f32(o[db][4 * jb] * inv) |
                          ((uint32_t)elem<T>::from_f32(o[db][4 * jb + 1] * inv) << 16);
      const uint32_t w1 = (uint32_t)elem<T>::from_f32(o[db][4 * jb + 2] * inv) |
                          ((uint32_t)elem<T>::from_f32(o[db][4 * jb + 3] * inv) << 16);
      *reinterpret_cast<uint2*>(orow + d0) = make_uint2(w0, w1);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

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
  const int eb = dtype_bytes(dtype);
  if ((dtype == RG_DTYPE_BF16 || dtype == RG_DTYPE_F16) && num_heads == 4 * num_kv_heads &&
      (head_dim == 64 || head_dim == 128) && max_blocks_per_seq > 0 && aligned16(query) &&
      aligned16(key_cache) && aligned16(value_cache) && (stride * eb) % 16 == 0 &&
      (reinterpret_cast<uintptr_t>(output) & 7u) == 0) {
    // Upper bound of the number of 32-query tiles: every sequence adds at most one partial.
    const int64_t tiles = (int64_t)(num_tokens + kPT - 1) / kPT + num_seqs;
    const dim3 grid((unsigned)(tiles * num_kv_heads));
    auto go = [&](auto tag, auto dtag) {
      using T = decltype(tag);
      constexpr int D = decltype(dtag)::value;
      hipLaunchKernelGGL((prefill_mfma_kernel<T, D>), grid, dim3(kPThreads), 0, s, a,
                         static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key_cache),
                         static_cast<const uint16_t*>(value_cache), block_table, context_lens, cu_seqlens);
    };
    using D64 = std::integral_constant<int, 64>;
    using D128 = std::integral_constant<int, 128>;
    if (dtype == RG_DTYPE_BF16) {
      if (head_dim == 128) go(bf16_t{}, D128{});
      else go(bf16_t{}, D64{});
    } else {
      if (head_dim == 128) go(f16_t{}, D128{});
      else go(f16_t{}, D64{});
    }
    return check_launch(op);
  }
  return dispatch_dtype(dtype, [&](auto tag) {
    hipLaunchKernelGGL(prefill_generic_kernel<decltype(tag)>, dim3(num_tokens, num_heads), dim3(64),
                       0, s, a);
    return check_launch(op);
  });
}
