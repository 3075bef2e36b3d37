// Paged decode attention (one query token per sequence) for gfx950.
//
// Two partition kernels share one contract.  A workgroup handles one
// (partition p, kv-head, sequence) work item; partition p covers context
// tokens [p*P, min((p+1)*P, ctx)).  Depending on `mode` it writes
//   MODE_FINAL  : the normalised output (the grid has one partition per sequence)
//   MODE_PARTIAL: the unnormalised partial  tmp_out / exp_sums / max_logits
//                 (crates/vllm-cuda/src/kernels/paged_attention_v2_partition.cu:95-106)
//   MODE_AUTO   : MODE_FINAL for sequences that fit one partition, MODE_PARTIAL
//                 otherwise; the merge kernel then skips the single-partition ones.
//
// * decode_mfma_kernel (bf16/f16, head_dim 64/128/256, block_size 16 << j; 16-token
//   sub-blocks of larger blocks): the GQA group's query heads are replicated into the 16 rows
//   of a v_mfma_f32_16x16x32 A operand, each 16-token K sub-block is the B operand, so one K/V
//   block is read from HBM once per kv-head for all of its q-heads.
//   Scores go through an exp2 online softmax whose max is shared by the whole
//   wave (DPP row reductions), P.V runs on the VALU in fp32 with 16-byte V
//   loads, and four waves split the partition's blocks and merge through LDS.
// * decode_generic_kernel: any dtype (fp32 included), head_dim % 4 == 0 up to
//   256, any block size and GQA ratio; one wave per (partition, q-head, seq),
//   each lane owning 4 dims.  Used where the MFMA kernel does not apply.
//
// decode_merge_kernel combines the partials of one (seq, q-head):
//   M = max_p m_p, out = sum_p e^(m_p-M) tmp_p / sum_p e^(m_p-M) l_p
// (crates/vllm-cuda/src/kernels/paged_attention_v2_reduce.cu:50-95).
#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <utility>

#include "rg_common.hpp"

namespace rg {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

enum DecodeMode : int32_t { MODE_FINAL = 0, MODE_PARTIAL = 1, MODE_AUTO = 2 };

struct DecodeArgs {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_table;
  const int32_t* context_lens;
  void* out;
  float* tmp_out;
  float* exp_sums;
  float* max_logits;
  float scale_log2;  // scale * log2(e)
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t block_size;
  int32_t max_blocks;
  int32_t num_partitions;  // stride of the partial arrays
  int32_t partition_size;  // tokens per partition
  int64_t kv_stride;       // elements between blocks
  int32_t mode;
  // block_size = 16 << bs_shift for the MFMA and stream-K kernels (-1: another size).  They work
  // in 16-token sub-blocks: sub-block b of a sequence is rows 16 (b & mask) .. of the kv-head's
  // slice of physical block table[b >> bs_shift].
  int32_t bs_shift;
};

__device__ __forceinline__ int num_parts_for(int ctx, int P) { return (ctx + P - 1) / P; }

// ------------------------------------------------------------- generic ------

template <typename T>
__global__ __launch_bounds__(64) void decode_generic_kernel(DecodeArgs a) {
  using E = elem<T>;
  using S = typename E::storage;
  const int p = blockIdx.x;
  const int h = blockIdx.y;
  const int s = blockIdx.z;
  const int lane = threadIdx.x;
  // Contexts longer than the block table row are clamped to it, negative ones to 0.
  const int ctx = max(0, min(a.context_lens[s], a.max_blocks * a.block_size));
  const int P = a.partition_size;
  const int np_s = min(num_parts_for(ctx, P), a.num_partitions);
  const int D = a.head_dim;
  const bool final_out = a.mode == MODE_FINAL || (a.mode == MODE_AUTO && np_s <= 1);

  if (p >= np_s) {
    // Empty context: the single-pass kernels leave zeros
    // (paged_attention_v1_plus.cu:38 on a zero-filled output).
    if (ctx == 0 && p == 0 && final_out) {
      S* o = static_cast<S*>(a.out) + ((int64_t)s * a.num_heads + h) * D;
      for (int d = lane; d < D; d += 64) E::store(o, d, 0.f);
    }
    return;
  }
  const int kvh = h / (a.num_heads / a.num_kv_heads);
  const int d0 = lane * 4;
  const bool act = d0 < D;
  const S* qp = static_cast<const S*>(a.q) + ((int64_t)s * a.num_heads + h) * D;
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
  const int t1 = min(ctx, (p + 1) * P);
  for (int t = p * P; t < t1; ++t) {
    const int64_t blk = bt[t / a.block_size];
    const int off = t % a.block_size;
    const int64_t row = blk * a.kv_stride + ((int64_t)kvh * a.block_size + off) * D;
    float kv[4] = {0.f, 0.f, 0.f, 0.f}, vv[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        kv[u] = E::load(kc, row + d0 + u);
        vv[u] = E::load(vc, row + d0 + u);
      }
    }
    float dot = qv[0] * kv[0] + qv[1] * kv[1] + qv[2] * kv[2] + qv[3] * kv[3];
    dot = wave_sum(dot);
    const float x = dot * a.scale_log2;
    const float m_new = fmaxf(m, x);
    const float alpha = exp2f(m - m_new);
    const float pe = exp2f(x - m_new);
    l = l * alpha + pe;
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = o[u] * alpha + pe * vv[u];
    m = m_new;
  }

  if (final_out) {
    const float inv = l != 0.f ? 1.f / l : 1.f;
    S* op = static_cast<S*>(a.out) + ((int64_t)s * a.num_heads + h) * D;
    if (act) {
#pragma unroll
      for (int u = 0; u < 4; ++u) E::store(op, d0 + u, o[u] * inv);
    }
  } else {
    const int64_t sh = ((int64_t)s * a.num_heads + h) * a.num_partitions + p;
    if (act) {
      float4* tp = reinterpret_cast<float4*>(a.tmp_out + sh * D + d0);
      *tp = make_float4(o[0], o[1], o[2], o[3]);
    }
    if (lane == 0) {
      a.exp_sums[sh] = l;
      a.max_logits[sh] = m * kLn2;
    }
  }
}

// ---------------------------------------------------------------- MFMA ------

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct mfma16;
template <> struct mfma16<bf16_t> {
  __device__ static __forceinline__ f32x4_t run(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ void unpack8(uint4 u, float* f) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <> struct mfma16<f16_t> {
  __device__ static __forceinline__ f32x4_t run(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ void unpack8(uint4 u, float* f) {
    const f16x8_t h = __builtin_bit_cast(f16x8_t, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
  }
};

// DPP helpers: `ctrl` is a DPP control word (quad_perm / row_ror).  Every lane of the
// patterns used here has a valid source lane, so no "old" value is needed.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
// Max / sum over the 16 lanes of a row, result in every lane of the row.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp<0x128>(v));  // row_ror:8
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x124>(v);
  v += dpp<0x128>(v);
  return v;
}

// Orders LDS writes of one lane before LDS reads of another lane of the same wave: waits
// for the wave's LDS operations only (global loads in flight stay in flight) and keeps the
// compiler from moving memory accesses across.
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// 2^x with the hardware v_exp_f32 (results below 2^-126 flush to zero, which only drops
// softmax weights that are already negligible).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr int kBS = 16;  // tokens per KV block on the MFMA path

// Tuning knobs of the MFMA path (compile-time): waves per workgroup, blocks each wave keeps
// in flight ahead of the one it computes, and an optional occupancy floor.
#ifndef RG_DEC_WAVES
#define RG_DEC_WAVES 4
#endif
#ifndef RG_DEC_PREFETCH
#define RG_DEC_PREFETCH 1
#endif
constexpr int kWaves = RG_DEC_WAVES;
constexpr int kPrefetch = RG_DEC_PREFETCH;
constexpr int kThreads = kWaves * 64;
#if defined(RG_DEC_WAVES_PER_EU) && RG_DEC_WAVES_PER_EU > 0
#define RG_DEC_OCCUPANCY __attribute__((amdgpu_waves_per_eu(RG_DEC_WAVES_PER_EU)))
#else
#define RG_DEC_OCCUPANCY
#endif

// Online-softmax update of one step of NB blocks, shared by the decode tiles.  c[b] holds the
// raw scores of block b in the MFMA output layout (lane (col, seg): token col, heads 4*seg + r);
// tokens at context index >= ctx are masked.  Updates the wave-uniform running max m_run and
// the per-lane sums l_run (exp2 domain), writes the probabilities of the NB * 16 tokens to
// p_lds ([token][GP heads]) and the rescale factors to alpha_lds, and returns whether any
// head's maximum moved (then acc needs the rescale).
template <int NB, int GP, int HG>
__device__ __forceinline__ bool softmax_block(const f32x4_t (&c)[NB], int col, int seg, int tok0, int ctx,
                                              float scale_log2, float (&m_run)[4], float (&l_run)[4],
                                              float* p_lds, float* alpha_lds) {
  float x[NB][4];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const bool valid = tok0 + b * kBS + col < ctx;
#pragma unroll
    for (int r = 0; r < 4; ++r) x[b][r] = valid ? c[b][r] * scale_log2 : -INFINITY;
  }
  float pr[NB][4], al[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float mx = x[0][r];
#pragma unroll
    for (int b = 1; b < NB; ++b) mx = fmaxf(mx, x[b][r]);
    const float bm = row16_max(mx);
    const float m_new = fmaxf(m_run[r], bm);
    al[r] = fast_exp2(m_run[r] - m_new);
#pragma unroll
    for (int b = 0; b < NB; ++b) pr[b][r] = fast_exp2(x[b][r] - m_new);
    float ps = pr[0][r];
#pragma unroll
    for (int b = 1; b < NB; ++b) ps += pr[b][r];
    l_run[r] = l_run[r] * al[r] + ps;
    m_run[r] = m_new;
  }
  // The running max of a head moves on few blocks only: skip the rescale of acc when it
  // moved for no head (a wave-uniform decision).
  const bool rescale = __ballot(al[0] != 1.f || al[1] != 1.f || al[2] != 1.f || al[3] != 1.f) != 0;
  if (seg < HG) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
      *reinterpret_cast<float4*>(&p_lds[(b * kBS + col) * GP + 4 * seg]) =
          make_float4(pr[b][0], pr[b][1], pr[b][2], pr[b][3]);
    if (col == 0) *reinterpret_cast<float4*>(&alpha_lds[4 * seg]) = make_float4(al[0], al[1], al[2], al[3]);
  }
  wave_lds_sync();
  return rescale;
}

// Per-wave state and block step of the MFMA decode path, shared by the grid kernel and the
// stream-K kernel.  One wave owns one (sequence, kv-head) segment at a time and processes
// 16-token blocks:
//   QK role (MFMA): lane (col = lane%16, seg = lane/16) holds K[col][seg*D/4 ...] and the
//     q rows replicated so that MFMA row m is head m % G; the result gives every lane the
//     scores of 4 heads (rows 4*seg+r) for token `col`.
//   PV role (VALU): lane (vrow = lane/ROWV, vd0 = 8*(lane%ROWV)) holds V rows vrow + i*TPI,
//     dims vd0..vd0+8, and accumulates acc[h][0..8) for all G heads.
// The softmax runs in the exp2 domain with a wave-uniform running max per head; the
// probabilities travel from the QK layout to the PV layout through a small LDS area.
// Fused RoPE (decode_stream_kernel with ROPE): a lane's run of P consecutive rotation pairs
// (x[d + j], x[d + D/2 + j]), j < P, of one row, with their cos / sin, rotated with the arithmetic
// of the RoPE + cache pass (rope_chunk16: rope_rotate_pair, then one rounding to T) into an LDS
// row (p points into LDS).  Spreading a row's D/2 pairs over the lanes keeps the rotation to a
// few instructions per wave; the MFMA layouts read the rotated rows back from LDS.
template <int P>
__device__ __forceinline__ void load_u16(const uint16_t* p, uint16_t (&o)[P]) {
  if constexpr (P == 1) {
    o[0] = *p;
  } else {
    uint32_t w[P / 2];
    if constexpr (P == 2) {
      w[0] = *reinterpret_cast<const uint32_t*>(p);
    } else if constexpr (P == 4) {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      w[0] = v.x;
      w[1] = v.y;
    } else {
      static_assert(P == 8, "runs of 1, 2, 4 or 8 pairs");
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      w[0] = v.x;
      w[1] = v.y;
      w[2] = v.z;
      w[3] = v.w;
    }
#pragma unroll
    for (int j = 0; j < P / 2; ++j) {
      o[2 * j] = (uint16_t)(w[j] & 0xffffu);
      o[2 * j + 1] = (uint16_t)(w[j] >> 16);
    }
  }
}
template <int P>
__device__ __forceinline__ void store_u16(uint16_t* p, const uint16_t (&x)[P]) {
  if constexpr (P == 1) {
    *p = x[0];
  } else {
    uint32_t w[P / 2];
#pragma unroll
    for (int j = 0; j < P / 2; ++j) w[j] = (uint32_t)x[2 * j] | ((uint32_t)x[2 * j + 1] << 16);
    if constexpr (P == 2) *reinterpret_cast<uint32_t*>(p) = w[0];
    else if constexpr (P == 4) *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}
template <int P>
__device__ __forceinline__ void load_f32(const float* p, float (&o)[P]) {
  if constexpr (P == 1) {
    o[0] = *p;
  } else if constexpr (P == 2) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    o[0] = v.x;
    o[1] = v.y;
  } else {
#pragma unroll
    for (int j = 0; j < P; j += 4) {
      const float4 v = *reinterpret_cast<const float4*>(p + j);
      o[j] = v.x;
      o[j + 1] = v.y;
      o[j + 2] = v.z;
      o[j + 3] = v.w;
    }
  }
}
template <typename T, int P>
struct RopeRun {
  uint16_t lo[P], hi[P];
  float c[P], s[P];
  // row, cs: the row and its cos_sin row; d: the run's first pair; half = D / 2.
  __device__ __forceinline__ void load(const uint16_t* row, const float* cs, int d, int half) {
    load_u16<P>(row + d, lo);
    load_u16<P>(row + half + d, hi);
    load_f32<P>(cs + d, c);
    load_f32<P>(cs + half + d, s);
  }
  // The rounding is pack2's (v_cvt_pk_*: round to nearest even, two values per instruction),
  // which gives the bits of the pass's elem<T>::from_f32 for every value but NaN payloads.
  __device__ __forceinline__ void rotate_to(uint16_t* dst, int d, int half) const {
    using E = elem<T>;
    float fl[P], fh[P];
#pragma unroll
    for (int j = 0; j < P; ++j) rope_rotate_pair(E::to_f32(lo[j]), E::to_f32(hi[j]), c[j], s[j], fl[j], fh[j]);
    uint16_t ol[P], oh[P];
    if constexpr (P == 1) {
      const uint32_t w = pack2<T>(fl[0], fh[0]);
      ol[0] = (uint16_t)(w & 0xffffu);
      oh[0] = (uint16_t)(w >> 16);
    } else {
#pragma unroll
      for (int j = 0; j < P; j += 2) {
        const uint32_t wl = pack2<T>(fl[j], fl[j + 1]), wh = pack2<T>(fh[j], fh[j + 1]);
        ol[j] = (uint16_t)(wl & 0xffffu);
        ol[j + 1] = (uint16_t)(wl >> 16);
        oh[j] = (uint16_t)(wh & 0xffffu);
        oh[j + 1] = (uint16_t)(wh >> 16);
      }
    }
    store_u16<P>(dst + d, ol);
    store_u16<P>(dst + half + d, oh);
  }
};

template <typename T, int D, int G>
struct DecodeTile {
  using MF = mfma16<T>;
  using S = uint16_t;
  static constexpr int NK = D / 32;         // MFMAs (and 16-byte K loads) per block
  static constexpr int ROWV = D / 8;        // 16-byte vectors per token row
  static constexpr int TPI = 64 / ROWV;     // tokens covered by one V load instruction
  static constexpr int NV = kBS / TPI;      // V loads per block
  static constexpr int HG = (G + 3) / 4;    // MFMA output row groups (4 rows each) holding distinct heads
  // Heads per LDS row, padded to whole row groups: the softmax writes 4 rows per group, so for
  // G not a multiple of 4 (3, 5, 6, 7) the last group's rows past G (copies of heads m % G)
  // land in padding instead of the next token's row.
  static constexpr int GP = 4 * HG;
  static constexpr int ACC = 8;             // output dims per lane and head (acc[h][0..ACC))

  int col, seg, vrow, vd0;
  uint4 qa[NK];
  float m_run[4], l_run[4];
  float acc[G][8];

  __device__ __forceinline__ void init(int lane) {
    col = lane & 15;
    seg = lane >> 4;
    vrow = lane / ROWV;
    vd0 = (lane % ROWV) * 8;
  }
  // q rows of the G heads of one kv-head ([G, D] contiguous).  MFMA i takes dims
  // [32i, 32i + 32): lane (col, seg) holds dims 32i + 8seg .. +8 of head col % G.
  __device__ __forceinline__ void load_q(const S* qg) {
    const uint4* qrow = reinterpret_cast<const uint4*>(qg + (int64_t)(col % G) * D + seg * 8);
#pragma unroll
    for (int i = 0; i < NK; ++i) qa[i] = qrow[4 * i];
  }
  // Puts token `tok` of block `blk` of a loaded NB-block unit to the given K row (kn, load_row's
  // layout) and V piece (vn: dims vd0 .. vd0 + 8 of the row), as if they had been read from the
  // cache.  Register selects only: the entries stay at compile-time indices.
  template <int NB>
  __device__ __forceinline__ void patch(uint4 (&kk)[NB * NK], uint4 (&vv)[NB * NV], int blk, int tok,
                                        const uint4 (&kn)[NK], uint4 vn) const {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const bool kr = b == blk && col == tok;
#pragma unroll
      for (int i = 0; i < NK; ++i) {
        const uint4 o = kk[b * NK + i];
        kk[b * NK + i] = make_uint4(kr ? kn[i].x : o.x, kr ? kn[i].y : o.y, kr ? kn[i].z : o.z, kr ? kn[i].w : o.w);
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const bool vr = b == blk && i * TPI + vrow == tok;
        const uint4 o = vv[b * NV + i];
        vv[b * NV + i] = make_uint4(vr ? vn.x : o.x, vr ? vn.y : o.y, vr ? vn.z : o.z, vr ? vn.w : o.w);
      }
    }
  }
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m_run[r] = -INFINITY;
      l_run[r] = 0.f;
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }
  // kb / vb: the [16, D] rows of one kv-head in one block.
  // Load i of K reads dims 32i .. 32i + 32 of all 16 rows: 64 contiguous bytes per row.
  __device__ __forceinline__ void load(const S* kb, const S* vb, uint4 (&kk)[NK], uint4 (&vv)[NV]) const {
    load_part<1, 0>(kb, vb, kk, vv);
  }
  // load(), or with live == false the same number of load instructions, each reading the first
  // 16 bytes of kb (of vb) in every lane: one line per instruction instead of 16 rows.  A
  // pipeline that issues a fixed number of loads per step (so that the compiler's waits are
  // exact counts) fills its slots past the last block this way.
  __device__ __forceinline__ void load_or_line(const S* kb, const S* vb, bool live, uint4 (&kk)[NK],
                                               uint4 (&vv)[NV]) const {
    const int lm = live ? -1 : 0;
    const uint4* kp = reinterpret_cast<const uint4*>(kb + ((col * D + seg * 8) & lm));
#pragma unroll
    for (int i = 0; i < NK; ++i) kk[i] = stream_load16(kp + ((4 * i) & lm));
#pragma unroll
    for (int i = 0; i < NV; ++i) vv[i] = stream_load16(vb + (((i * TPI + vrow) * D + vd0) & lm));
  }
  // The same into entries [B*NK, (B+1)*NK) and [B*NV, (B+1)*NV) of an NB-block ring slot.
  template <int NB, int B>
  __device__ __forceinline__ void load_part(const S* kb, const S* vb, uint4 (&kk)[NB * NK], uint4 (&vv)[NB * NV]) const {
    const uint4* kp = reinterpret_cast<const uint4*>(kb + col * D + seg * 8);
#pragma unroll
    for (int i = 0; i < NK; ++i) kk[B * NK + i] = stream_load16(kp + 4 * i);
#pragma unroll
    for (int i = 0; i < NV; ++i) vv[B * NV + i] = stream_load16(vb + (i * TPI + vrow) * D + vd0);
  }
  // NB consecutive blocks of one kv-head (kr / vr: block b in entries [b*NK, (b+1)*NK) and
  // [b*NV, (b+1)*NV)) whose first token has context index tok0; tokens >= ctx are masked.  One
  // running-max update, rescale decision and LDS exchange serve all NB * 16 tokens.
  // p_lds holds NB * 16 rows of GP probabilities.
  template <int NB = 1>
  __device__ __forceinline__ void step(const uint4 (&kr)[NB * NK], const uint4 (&vr)[NB * NV], int tok0, int ctx,
                                       float scale_log2, float* p_lds, float* alpha_lds) {
    f32x4_t c[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      c[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < NK; ++i) c[b] = MF::run(qa[i], kr[b * NK + i], c[b]);
    }
    const bool tail = tok0 + NB * kBS > ctx;
    const bool rescale = softmax_block<NB, GP, HG>(c, col, seg, tok0, ctx, scale_log2, m_run, l_run, p_lds, alpha_lds);
    if (rescale) {
      float alh[G];
#pragma unroll
      for (int h = 0; h < G; ++h) alh[h] = alpha_lds[h];
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] *= alh[h];
    }
    // V load i covers tokens i * TPI .. + TPI of the NB * 16 (NV * TPI = 16 per block).
    float vf[NB * NV][8];
#pragma unroll
    for (int i = 0; i < NB * NV; ++i) MF::unpack8(vr[i], vf[i]);
    if (tail) {
      // Rows past the context may hold any bit pattern; keep them out of 0*x.
#pragma unroll
      for (int i = 0; i < NB * NV; ++i) {
        if (tok0 + i * TPI + vrow >= ctx) {
#pragma unroll
          for (int e = 0; e < 8; ++e) vf[i][e] = 0.f;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NB * NV; ++i) {
      const int t = i * TPI + vrow;
      float ph[G];
#pragma unroll
      for (int h = 0; h < G; ++h) ph[h] = p_lds[t * GP + h];
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] += ph[h] * vf[i][e];
    }
  }
  // Sums acc over the TPI token rows (result valid in lanes with vrow == 0) and l over the
  // 16 columns (lsum[r] for head 4*seg+r, valid in every lane).
  __device__ __forceinline__ void reduce(float (&lsum)[4]) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = acc[h][e];
#pragma unroll
        for (int o = ROWV; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
        acc[h][e] = v;
      }
#pragma unroll
    for (int r = 0; r < 4; ++r) lsum[r] = row16_sum(l_run[r]);
  }
};

// The fp32 tile (the reference's own element type): the same per-wave state and step as
// DecodeTile, with QK^T on v_mfma_f32_16x16x4_f32.  MFMA m of a block takes the k-slot s of
// lane (col, seg) from dim DQ*s + m (DQ = D/4), so lane (col, seg) holds the contiguous run
// K[col][DQ*seg .. DQ*seg + DQ) (DQ/4 16-byte loads) and, as the A operand, the same dims of
// head col % G; the output has DecodeTile's layout (scores of heads 4*seg + r for token col),
// so the softmax is softmax_block.  P.V runs on the VALU with 16-byte fp32 V loads: lane
// (vrow, vd0) holds 4 dims of V rows vrow + i*TPI.
template <int D, int G>
struct DecodeTileF32 {
  using S = float;
  static constexpr int DQ = D / 4;          // dims per lane in QK (and MFMAs per block)
  static constexpr int NK = DQ / 4;         // 16-byte K loads per block
  static constexpr int ROWV = D / 4;        // 16-byte vectors per token row
  static constexpr int TPI = 64 / ROWV;     // tokens covered by one V load instruction
  static constexpr int NV = kBS / TPI;      // V loads per block
  static constexpr int HG = (G + 3) / 4;
  static constexpr int GP = 4 * HG;  // as DecodeTile
  static constexpr int ACC = 4;
  static_assert(NK >= 1 && TPI >= 1 && NV >= 1, "head_dim 64, 128 or 256");

  int col, seg, vrow, vd0;
  float qa[DQ];
  float m_run[4], l_run[4];
  float acc[G][4];

  __device__ __forceinline__ void init(int lane) {
    col = lane & 15;
    seg = lane >> 4;
    vrow = lane / ROWV;
    vd0 = (lane % ROWV) * 4;
  }
  __device__ __forceinline__ void load_q(const float* qg) {
    const float4* qrow = reinterpret_cast<const float4*>(qg + (int64_t)(col % G) * D + seg * DQ);
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const float4 v = qrow[i];
      qa[4 * i] = v.x;
      qa[4 * i + 1] = v.y;
      qa[4 * i + 2] = v.z;
      qa[4 * i + 3] = v.w;
    }
  }
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m_run[r] = -INFINITY;
      l_run[r] = 0.f;
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[h][e] = 0.f;
  }
  template <int NB, int B>
  __device__ __forceinline__ void load_part(const float* kb, const float* vb, uint4 (&kk)[NB * NK],
                                            uint4 (&vv)[NB * NV]) const {
    // K with ordinary loads (a lane's eight K loads cover one line in 16-byte steps: with the
    // non-temporal hint the tile ran 1.6x slower, 332 against 209 us at config 2's shape), V
    // streamed (208 -> 188 us).
    const uint4* kp = reinterpret_cast<const uint4*>(kb + col * D + seg * DQ);
#pragma unroll
    for (int i = 0; i < NK; ++i) kk[B * NK + i] = kp[i];
#pragma unroll
    for (int i = 0; i < NV; ++i) vv[B * NV + i] = stream_load16(vb + (i * TPI + vrow) * D + vd0);
  }
  __device__ __forceinline__ void load(const float* kb, const float* vb, uint4 (&kk)[NK], uint4 (&vv)[NV]) const {
    load_part<1, 0>(kb, vb, kk, vv);
  }
  template <int NB = 1>
  __device__ __forceinline__ void step(const uint4 (&kr)[NB * NK], const uint4 (&vr)[NB * NV], int tok0, int ctx,
                                       float scale_log2, float* p_lds, float* alpha_lds) {
    f32x4_t c[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      c[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < NK; ++i) {
        const uint4 k4 = kr[b * NK + i];
        const uint32_t kw[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          c[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * i + e], __uint_as_float(kw[e]), c[b], 0, 0, 0);
      }
    }
    const bool tail = tok0 + NB * kBS > ctx;
    const bool rescale = softmax_block<NB, GP, HG>(c, col, seg, tok0, ctx, scale_log2, m_run, l_run, p_lds, alpha_lds);
    if (rescale) {
      float alh[G];
#pragma unroll
      for (int h = 0; h < G; ++h) alh[h] = alpha_lds[h];
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[h][e] *= alh[h];
    }
#pragma unroll
    for (int i = 0; i < NB * NV; ++i) {
      const int t = i * TPI + vrow;
      float vf[4] = {__uint_as_float(vr[i].x), __uint_as_float(vr[i].y), __uint_as_float(vr[i].z),
                     __uint_as_float(vr[i].w)};
      if (tail && tok0 + t >= ctx) {
        // Rows past the context may hold any bit pattern; keep them out of 0*x.
#pragma unroll
        for (int e = 0; e < 4; ++e) vf[e] = 0.f;
      }
      float ph[G];
#pragma unroll
      for (int h = 0; h < G; ++h) ph[h] = p_lds[t * GP + h];
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[h][e] += ph[h] * vf[e];
    }
  }
  __device__ __forceinline__ void reduce(float (&lsum)[4]) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[h][e];
#pragma unroll
        for (int o = ROWV; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
        acc[h][e] = v;
      }
#pragma unroll
    for (int r = 0; r < 4; ++r) lsum[r] = row16_sum(l_run[r]);
  }
};

// The tile type of element type T.
template <typename T, int D, int G>
using DecodeTileFor = std::conditional_t<std::is_same_v<T, f32_t>, DecodeTileF32<D, G>, DecodeTile<T, D, G>>;

// Grid decomposition: workgroup = (partition p, kv-head, sequence), kWaves waves taking the
// partition's blocks round-robin, merged through LDS at the end.
template <typename T, int D, int G>
__global__ __launch_bounds__(kThreads) RG_DEC_OCCUPANCY void decode_mfma_kernel(
    DecodeArgs a, const uint16_t* __restrict__ q_ptr, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ context_lens) {
  using Tile = DecodeTile<T, D, G>;
  using S = uint16_t;
  constexpr int GP = Tile::GP;
  constexpr int HG = Tile::HG;
  constexpr int NK = Tile::NK;
  constexpr int NV = Tile::NV;
  constexpr int NBUF = kPrefetch + 1;

  __shared__ float p_lds[kWaves][2][kBS * GP];
  __shared__ float alpha_lds[kWaves][2][GP];
  __shared__ float acc_lds[kWaves][G * D];
  __shared__ float ml_lds[kWaves][2][GP];

  const int p = blockIdx.x;
  const int kvh = blockIdx.y;
  const int s = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int ctx = max(0, min(context_lens[s], a.max_blocks * a.block_size));
  const int P = a.partition_size;
  const int np_s = min(num_parts_for(ctx, P), a.num_partitions);
  const bool final_out = a.mode == MODE_FINAL || (a.mode == MODE_AUTO && np_s <= 1);
  const int H = a.num_heads;

  if (p >= np_s) {
    if (ctx == 0 && p == 0 && final_out) {
      S* o = static_cast<S*>(a.out) + ((int64_t)s * H + (int64_t)kvh * G) * D;
      for (int i = tid; i < G * D; i += kThreads) o[i] = 0;
    }
    return;
  }

  // 16-token sub-blocks of this partition; wave w takes sub-blocks b0+w, b0+w+kWaves, ...
  const int nblk_ctx = (ctx + kBS - 1) / kBS;
  const int b0 = p * (P / kBS);
  const int b1 = min(nblk_ctx, b0 + P / kBS);
  const int nb = b0 + w < b1 ? (b1 - (b0 + w) + kWaves - 1) / kWaves : 0;

  Tile tile;
  tile.init(lane);
  tile.load_q(q_ptr + ((int64_t)s * H + (int64_t)kvh * G) * D);
  tile.reset();
  const int32_t* bt = block_table + (int64_t)s * a.max_blocks;
  const int64_t head_off = (int64_t)kvh * a.block_size * D;
  const int sh = a.bs_shift, sub_mask = (1 << sh) - 1;
  // Block j of this wave, or (j >= nb) one line of its last block per load instruction.
  auto load_block = [&](int j, uint4 (&kk)[NK], uint4 (&vv)[NV]) {
    const int lb = b0 + w + min(j, nb - 1) * kWaves;
    const int64_t off = (int64_t)bt[lb >> sh] * a.kv_stride + head_off + (int64_t)(lb & sub_mask) * (kBS * D);
    tile.load_or_line(kc + off, vc + off, j < nb, kk, vv);
  };

  // Software pipeline: kPrefetch blocks in flight ahead of the one being computed.  Every
  // step issues the same load instructions, so the waits stay exact counts instead of full
  // drains; past the end they read one line of the wave's last block each (a re-read of the
  // whole block was 1 in 8 of a P = 512 partition's requests).
  uint4 kbuf[NBUF][NK], vbuf[NBUF][NV];
  if (nb > 0) {
#pragma unroll
    for (int u = 0; u < kPrefetch; ++u) load_block(u, kbuf[u], vbuf[u]);
  }
  for (int j0 = 0; j0 < nb; j0 += NBUF) {
#pragma unroll
    for (int u = 0; u < NBUF; ++u) {
      const int j = j0 + u;
      if (j < nb) {
        load_block(j + kPrefetch, kbuf[(u + kPrefetch) % NBUF], vbuf[(u + kPrefetch) % NBUF]);
        tile.step(kbuf[u], vbuf[u], (b0 + w + j * kWaves) * kBS, ctx, a.scale_log2, p_lds[w][j & 1],
                  alpha_lds[w][j & 1]);
      }
    }
  }

  float lsum[4];
  tile.reduce(lsum);
  if (tile.vrow == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float4* dst = reinterpret_cast<float4*>(&acc_lds[w][h * D + tile.vd0]);
      dst[0] = make_float4(tile.acc[h][0], tile.acc[h][1], tile.acc[h][2], tile.acc[h][3]);
      dst[1] = make_float4(tile.acc[h][4], tile.acc[h][5], tile.acc[h][6], tile.acc[h][7]);
    }
  }
  if (tile.seg < HG && tile.col == 0) {
    *reinterpret_cast<float4*>(&ml_lds[w][0][4 * tile.seg]) =
        make_float4(tile.m_run[0], tile.m_run[1], tile.m_run[2], tile.m_run[3]);
    *reinterpret_cast<float4*>(&ml_lds[w][1][4 * tile.seg]) = make_float4(lsum[0], lsum[1], lsum[2], lsum[3]);
  }
  __syncthreads();

  // Merge the waves and write out two consecutive dims per thread.
  for (int idx = tid; idx < G * D / 2; idx += kThreads) {
    const int h = idx / (D / 2);
    const int d = (idx % (D / 2)) * 2;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, ml_lds[ww][0][h]);
    float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      const float mw = ml_lds[ww][0][h];
      const float f = mw == -INFINITY ? 0.f : exp2f(mw - M);
      L += f * ml_lds[ww][1][h];
      o0 += f * acc_lds[ww][h * D + d];
      o1 += f * acc_lds[ww][h * D + d + 1];
    }
    const int hq = kvh * G + h;
    if (final_out) {
      const float inv = L != 0.f ? 1.f / L : 1.f;
      S* op = static_cast<S*>(a.out) + ((int64_t)s * H + hq) * D + d;
      const uint32_t packed = (uint32_t)elem<T>::from_f32(o0 * inv) |
                              ((uint32_t)elem<T>::from_f32(o1 * inv) << 16);
      *reinterpret_cast<uint32_t*>(op) = packed;
    } else {
      const int64_t sh = ((int64_t)s * H + hq) * a.num_partitions + p;
      *reinterpret_cast<float2*>(a.tmp_out + sh * D + d) = make_float2(o0, o1);
      if (d == 0) {
        a.exp_sums[sh] = L;
        a.max_logits[sh] = M * kLn2;
      }
    }
  }
}

// ------------------------------------------------------------- stream-K -----
//
// The decode work is the list of units (sequence s, kv-head, b) ordered with b fastest,
// unit b covering blocks [b * BPU, b * BPU + BPU) of the sequence (sk_bpu: 1 at head_dim 128,
// 4 at head_dim 64, 2 at head_dim 64 with G >= 8); segment g = s * num_kv_heads + kvh is the
// run of units of one (s, kv-head).
// Worker k (one wave) takes a contiguous range of the U units, the k-th of W equal shares of
// their cost (the units' bytes plus a fixed cost per segment start, see the kernel), so every
// wave streams the same work whatever the context lengths are.  A worker emits one partial
// (m, l, acc) for every segment it touches, at partial index k + g (distinct for all
// (worker, segment) pairs because each worker's segments and each segment's workers are
// consecutive).  decode_stream_merge_kernel combines the partials of each segment.  With few
// units only the first workers are used, so every worker of a segment's range owns units.

// Units in flight ahead of the one being computed, per stream-K worker.  The workers are
// one wave per SIMD (RG_SK_WAVES_PER_CU = 4): two waves sharing a SIMD progress at
// different rates (the older one wins issue arbitration), which leaves the younger half
// of a static split running alone at the end; one wave per SIMD with 8 KB units in flight
// streams at the same rate without that tail.  One ahead: with the non-temporal K/V loads and
// the cost split, paired runs against three ahead gave config 2 0.990 (twice) with two ahead and
// 0.993-0.995 more with one (config 3 0.992, then 0.995-0.996), four ahead 1.011; the 1,024
// workers keep ~16 MB in flight with one unit each ahead, more than the HBM round trip needs.
#ifndef RG_SK_PREFETCH
#define RG_SK_PREFETCH 1
#endif
#ifndef RG_SK_BPU_D128
#define RG_SK_BPU_D128 1
#endif
// Blocks per stream-K unit and prefetch depth at head_dim 64.  A block of one kv-head is
// 2 KB of K + 2 KB of V there, while the per-unit fixed work (running-max reductions,
// rescale decision, LDS exchange, cursor) is the same as at head_dim 128.  Units of four
// blocks (16 KB) with two of them in flight measured fastest: 206.6 us per layer at the
// Llama-3.2-1B step against 216.6 us for two-block units three deep and 236.5 us for
// one-block units four deep (2 x 4, 2 x 5 and 3 x 3 were in between), with ordinary K/V
// loads; with the non-temporal loads 4 x 2 stays ahead of 2 x 3 and 4 x 3 (194.7 against
// 196.0 / 198.0 us per call), and with the cost split 4 x 1 ahead of 4 x 2 (0.992-0.993 in
// paired runs at the Llama-3.2-1B attention shape).
#ifndef RG_SK_BPU_D64
#define RG_SK_BPU_D64 4
#endif
#ifndef RG_SK_PREFETCH_D64
#define RG_SK_PREFETCH_D64 1
#endif
// With 8 or more q-heads per kv-head the accumulators take 8 * G registers per lane, so at
// head_dim 64 the unit ring shrinks to two-block units (half the registers of the four-block
// ring, which G >= 8 fills to the limit).
template <int D, int G>
constexpr int sk_bpu() { return D <= 64 ? (G >= 8 ? 2 : RG_SK_BPU_D64) : RG_SK_BPU_D128; }
// head_dim 256 (bf16 / f16): one-block units of 16 KB (8 KB of K, 8 KB of V) two deep.
template <int D, int G>
constexpr int sk_prefetch() { return D <= 64 ? RG_SK_PREFETCH_D64 : D >= 256 ? 2 : RG_SK_PREFETCH; }
// fp32 rows are twice as long: one-block units (8 KB of K and of V at head_dim 128), one in
// flight ahead at head_dim 128 and 256 and two at head_dim 64 (the register ring of the 16-bit
// tiles' depth would not fit).
template <typename T, int D, int G>
constexpr int sk_bpu_for() { return std::is_same_v<T, f32_t> ? 1 : sk_bpu<D, G>(); }
template <typename T, int D, int G>
constexpr int sk_prefetch_for() { return std::is_same_v<T, f32_t> ? (D <= 64 ? 2 : 1) : sk_prefetch<D, G>(); }

// Optional occupancy floor of the stream-K kernel (waves per SIMD).
#if defined(RG_SK_OCC) && RG_SK_OCC > 0
#define RG_SK_OCCUPANCY __attribute__((amdgpu_waves_per_eu(RG_SK_OCC)))
#else
#define RG_SK_OCCUPANCY
#endif

struct StreamArgs {
  void* out;
  float* part_acc;   // [num_partials, G, D]
  float* part_ml;    // [num_partials, G, 2]: (m in log2 units, l)
  int2* seg_desc;    // [batch * H_kv]: (first worker, number of workers) of each segment with units
  float scale_log2;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t max_blocks;
  int32_t batch;
  int32_t num_workers;
  int64_t kv_stride;
  int32_t table_stride;  // entries per block-table row (max_blocks counts 16-token sub-blocks)
  int32_t bs_shift;      // block_size = 16 << bs_shift
  // Fused RoPE + cache write of the step's new tokens (decode_stream_kernel with ROPE): token s
  // is sequence s's; its k / v rows are [H_kv, D] at k_new / v_new + s H_kv D.
  const void* k_new;
  const void* v_new;
  const float* cos_sin;         // [positions, D]: cos at [d], sin at [D/2 + d]
  const int32_t* positions;     // [batch]
  const int32_t* slot_mapping;  // [batch]; negative: a padding token, not cached
};

// Cost of a segment start, in KB of K/V streaming.  A worker's end time tracks the segments it
// touches (per-worker timestamps at config 2, 1,024 workers of ~69 units: each extra segment
// start -- q load, partial write, the pipeline's restart -- ends the worker ~1.6 us later, about
// 10 KB of its stream), so the split evens out (unit KB) x units + RG_SK_SEG_COST_KB x segment
// starts instead of units alone.  0: units only.  Swept in paired runs against 10 (config 2 /
// the config-5 attention shape): 5 KB 0.999 / 1.012, 15 KB 0.996 / 0.997, 20 KB 0.988-0.993 /
// 0.999-1.000, 30 KB 1.002 / 1.003.
#ifndef RG_SK_SEG_COST_KB
#define RG_SK_SEG_COST_KB 20
#endif
// The same with the step's RoPE + cache pass fused in (its segment starts also rotate q).  Kept
// at RG_SK_SEG_COST_KB, so that the fused step splits the work as the decode alone does and its
// output equals the two-entry chain's bit for bit; swept in paired runs of the fused entry at
// config 2 against 20: 14 KB 1.004, 26 KB 0.996, 32 KB 0.999 (26 KB moves the split, and three
// of config 2's 98,304 outputs then differ from the chain's by 2 ulp).
#ifndef RG_SK_SEG_COST_KB_ROPE
#define RG_SK_SEG_COST_KB_ROPE RG_SK_SEG_COST_KB
#endif

// 16-token sub-blocks of sequence s: ceil(ctx/16) per kv-head (context clamped to the table
// row, max_blocks of them).
__device__ __forceinline__ int seq_blocks(const int32_t* ctxl, int s, int max_blocks) {
  const int c = max(0, min(ctxl[s], max_blocks * kBS));
  return (c + kBS - 1) / kBS;
}
// Stream-K units of sequence s per kv-head: its blocks in runs of BPU (the last run may be short).
template <int BPU>
__device__ __forceinline__ int seq_units(const int32_t* ctxl, int s, int max_blocks) {
  return (seq_blocks(ctxl, s, max_blocks) + BPU - 1) / BPU;
}

// A wave-uniform 64-bit value made visibly uniform to the compiler.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Wave-wide inclusive prefix sum.
__device__ __forceinline__ int64_t wave_incl_scan(int64_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// ROPE: the step's RoPE + cache pass fused in (16-bit tiles).  q is read unrotated and left
// so; every worker of a segment rotates its q rows itself, and the worker holding a segment's
// last unit rotates the new token's k row, writes k and v to the token's cache slot and puts
// them into its own loaded copy of that block in place of what the cache held.  No worker reads
// another's store, and the outputs and cache equal those of the RoPE + cache pass followed by
// the decode bit for bit.  positions / slot_mapping: [batch], token s being sequence s's.
template <typename T, int D, int G, bool ROPE = false>
__global__ __launch_bounds__(64) RG_SK_OCCUPANCY void decode_stream_kernel(
    StreamArgs a, const typename DecodeTileFor<T, D, G>::S* __restrict__ q_ptr,
    const typename DecodeTileFor<T, D, G>::S* __restrict__ kc, const typename DecodeTileFor<T, D, G>::S* __restrict__ vc,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ context_lens,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ slot_mapping) {
  using Tile = DecodeTileFor<T, D, G>;
  static_assert(!ROPE || !std::is_same_v<T, f32_t>, "the fused RoPE runs on the 16-bit tiles");
  constexpr int GP = Tile::GP;
  constexpr int HG = Tile::HG;
  constexpr int NK = Tile::NK;
  constexpr int NV = Tile::NV;
  constexpr int kSkPrefetch = sk_prefetch_for<T, D, G>();
  constexpr int NBUF = kSkPrefetch + 1;
  constexpr int BPU = sk_bpu_for<T, D, G>();
  __shared__ float p_lds[2][BPU * kBS * GP];
  __shared__ float alpha_lds[2][GP];

  const int lane = threadIdx.x;
  const int64_t k = blockIdx.x;
  const int hkv = a.num_kv_heads;
  // Total units U, this worker's range [u0, u1) and the sequence holding u0: one pass over
  // the context lengths for up to 64 sequences (one per lane), two for larger batches.
  //
  // The split evens out cost, not units: unit u of segment g (segments numbered over the
  // non-empty ones, in unit order) sits at z(u) = KQ u + KS (g + 1), KQ its K/V kilobytes and KS
  // a segment start's (RG_SK_SEG_COST_KB; with 0, KQ = 1 and the split is by units), and of the
  // total C = KQ U + KS S worker k takes the units with k C / W <= z(u) < (k + 1) C / W.
  // Consecutive z are at most KQ + KS apart, so with W <= C / (KQ + KS) every worker owns a unit
  // (with fewer units than workers, only the first workers run), as the merge's segment ranges
  // need.
  constexpr int64_t KS = ROPE ? RG_SK_SEG_COST_KB_ROPE : RG_SK_SEG_COST_KB;
  constexpr int64_t KQ = KS > 0 ? (int64_t)BPU * kBS * D * sizeof(typename Tile::S) * 2 / 1024 : 1;
  static_assert(KQ >= 1, "unit cost");
  int64_t C, W, u0, u1, seq_start;
  int s, seq_seg;  // the sequence holding u0 and the index of its first segment
  // Lanes below this one whose sequence has units (a sequence's segments all do or all don't).
  auto below = [&](bool f) __attribute__((always_inline)) -> int {
    const uint64_t m = __ballot(f);
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
  };
  // The first unit at or after cost x in a sequence of nb units per kv-head whose costs start
  // at cx and units at ex (j == nb: the next segment's first unit).  The offset into one
  // sequence fits 32 bits for any table the device holds; the division is done in 32 bits then.
  auto unit_in = [&](int64_t x, int64_t cx, int64_t ex, int64_t nb) __attribute__((always_inline)) -> int64_t {
    const int64_t seg = KS + KQ * nb, o = x - cx;
    const int64_t kv = (o >> 31) == 0 && (seg >> 31) == 0 ? (int64_t)((uint32_t)o / (uint32_t)seg) : o / seg;
    const int64_t r = o - kv * seg;
    const int64_t j = r <= KS ? 0 : (r - KS + KQ - 1) / KQ;
    return ex + kv * nb + j;
  };
  // k C / W in 32 bits when it fits.
  auto share = [&](int64_t kk) __attribute__((always_inline)) -> int64_t {
    const int64_t v = kk * C;
    return (v >> 32) == 0 ? (int64_t)((uint32_t)v / (uint32_t)W) : v / W;
  };
  {
    // First pass over the sequences, 64 per step: the totals U and C.  A batch of up to 64 keeps
    // its lane values (units n, inclusive unit scan, non-empty sequences below) for the second.
    int64_t U = 0, ne = 0, n1 = 0, incl1 = 0, nb1 = 0;
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
      const int q = c0 + lane;
      const int64_t n = q < a.batch ? (int64_t)seq_units<BPU>(context_lens, q, a.max_blocks) * hkv : 0;
      const int64_t incl = wave_incl_scan(n, lane) + U;
      if (c0 == 0) {
        n1 = n;
        incl1 = incl;
        nb1 = below(n > 0);
      }
      U = uniform64(__shfl(incl, 63, 64));
      ne += __builtin_popcountll(__ballot(n > 0));
    }
    C = KQ * U + KS * hkv * ne;
    W = min<int64_t>(a.num_workers, C / (KQ + KS));
    if (k >= W) return;
    // Second pass: the units at costs x0 = k C / W and x1 = (k + 1) C / W (the last worker ends at
    // U), and the sequence holding u0 with the index of its first segment.
    const int64_t x0 = share(k), x1 = k + 1 < W ? share(k + 1) : C;
    u0 = U;
    u1 = U;
    s = -1;
    seq_start = 0;
    seq_seg = 0;
    bool rolled = false;  // u0 is the first unit past the sequence whose costs hold x0
    bool need1 = x1 < C;
    auto resolve = [&](int c0, int64_t n, int64_t incl, int64_t nb_) __attribute__((always_inline)) {
      const int64_t excl = incl - n;
      const int64_t cexcl = KQ * excl + KS * hkv * nb_, cincl = cexcl + (n > 0 ? KQ * n + KS * hkv : 0);
      if (s < 0) {
        const uint64_t h = __ballot(n > 0 && cexcl <= x0 && x0 < cincl);
        if (h) {
          const int l = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)h) - 1);
          const int64_t el = uniform64(__shfl(excl, l, 64)), nl = uniform64(__shfl(n, l, 64));
          u0 = unit_in(x0, uniform64(__shfl(cexcl, l, 64)), el, nl / hkv);
          s = c0 + l;
          seq_start = el;
          seq_seg = (int)(hkv * uniform64(__shfl(nb_, l, 64)));
          rolled = u0 == el + nl;
        }
      }
      if (need1) {
        const uint64_t h = __ballot(n > 0 && cexcl <= x1 && x1 < cincl);
        if (h) {
          const int l = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)h) - 1);
          u1 = unit_in(x1, uniform64(__shfl(cexcl, l, 64)), uniform64(__shfl(excl, l, 64)),
                       uniform64(__shfl(n, l, 64)) / hkv);
          need1 = false;
        }
      }
    };
    if (a.batch <= 64) {
      resolve(0, n1, incl1, nb1);
    } else {
      int64_t ub = 0, nb = 0;
      for (int c0 = 0; c0 < a.batch && (s < 0 || need1); c0 += 64) {
        const int q = c0 + lane;
        const int64_t n = q < a.batch ? (int64_t)seq_units<BPU>(context_lens, q, a.max_blocks) * hkv : 0;
        const int64_t incl = wave_incl_scan(n, lane) + ub;
        resolve(c0, n, incl, nb + below(n > 0));
        ub = uniform64(__shfl(incl, 63, 64));
        nb += __builtin_popcountll(__ballot(n > 0));
      }
    }
    if (rolled) {
      // u0 is the first unit of a later sequence (a share boundary in the cost of a sequence's
      // last unit, past its start): find that sequence by units.
      int64_t ub = 0, nb = 0;
      s = -1;
      for (int c0 = 0; c0 < a.batch && s < 0; c0 += 64) {
        const int q = c0 + lane;
        const int64_t n = q < a.batch ? (int64_t)seq_units<BPU>(context_lens, q, a.max_blocks) * hkv : 0;
        const int64_t incl = wave_incl_scan(n, lane) + ub, excl = incl - n;
        const int64_t nb_ = nb + below(n > 0);
        const uint64_t h = __ballot(n > 0 && excl <= u0 && u0 < incl);
        if (h) {
          const int l = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)h) - 1);
          s = c0 + l;
          seq_start = uniform64(__shfl(excl, l, 64));
          seq_seg = (int)(hkv * uniform64(__shfl(nb_, l, 64)));
        }
        ub = uniform64(__shfl(incl, 63, 64));
        nb += __builtin_popcountll(__ballot(n > 0));
      }
    }
    s = __builtin_amdgcn_readfirstlane(s);
    seq_seg = __builtin_amdgcn_readfirstlane(seq_seg);
  }

  // Cursor of the unit being computed and of the unit being loaded: sequence, kv-head, unit b
  // of the segment's nblk units (blocks b * BPU .. b * BPU + BPU - 1).
  struct Cursor {
    int s, kvh, b, nblk;
  };
  // The cursors are wave-uniform; readfirstlane tells the compiler so (seq_start comes out of
  // a cross-lane shuffle), which keeps every block-table and context-length read a scalar
  // load instead of a vector load whose wait would also drain the K/V prefetches.
  Cursor cur;
  cur.s = s;
  cur.nblk = __builtin_amdgcn_readfirstlane(seq_units<BPU>(context_lens, s, a.max_blocks));
  {
    const int r = __builtin_amdgcn_readfirstlane((int)(u0 - seq_start));
    cur.kvh = __builtin_amdgcn_readfirstlane(r / cur.nblk);
    cur.b = __builtin_amdgcn_readfirstlane(r - cur.kvh * cur.nblk);
  }
  // Index g of the current segment among the non-empty ones (a sequence's costs start at
  // KQ x its first unit + KS x the segments before it), moved on at each segment end.
  int seg = seq_seg + cur.kvh;
  // Every lambda of the kernel is forced inline: one left out of line is called with its
  // captures in scratch memory (G = 16, and D = 64 with G = 8, spilled that way).
  auto advance = [&](Cursor& c) __attribute__((always_inline)) {
    if (++c.b == c.nblk) {
      c.b = 0;
      if (++c.kvh == hkv) {
        c.kvh = 0;
        do {
          ++c.s;
          c.nblk = c.s < a.batch ? seq_units<BPU>(context_lens, c.s, a.max_blocks) : 1;
        } while (c.nblk == 0);
      }
    }
  };
  // Block numbers of the worker's units in a register window: lane i holds the blocks of
  // unit wbase + i (units counted from u0; btw[r] is sub-block r of the unit as
  // (physical block << bs_shift) | sub-block within it, and a short last unit repeats its
  // first sub-block, which the step masks).  Filling it walks each lane's cursor
  // i units on (a few steps: ranges cross few segments) and reads all 64 units' entries with
  // BPU loads, so the per-unit address needs a v_readlane instead of a scalar load waited on
  // in the loop.
  int64_t wbase = 0;
  int btw[BPU];
  // ROPE: per window lane, the RoPE position of its unit's sequence (pwin) and, if the unit is its
  // segment's last and the sequence's slot is the block table's slot of position context_len - 1,
  // that slot (rwin; else -1).  Read with the block numbers, so no segment start waits on a
  // scalar load for them.
  int pwin = 0, rwin = -1;
  auto fill_window = [&](const Cursor& c0, int64_t base) __attribute__((always_inline)) {
    int ss = c0.s, kh = c0.kvh, b = c0.b + lane, nb = c0.nblk;
    while (b >= nb && ss < a.batch) {
      b -= nb;
      if (++kh == hkv) {
        kh = 0;
        do {
          ++ss;
          nb = ss < a.batch ? seq_units<BPU>(context_lens, ss, a.max_blocks) : 1;
        } while (nb == 0);
      }
    }
    const bool live = base + lane < u1 - u0 && ss < a.batch;
    const int32_t* row = block_table + (int64_t)(live ? ss : 0) * a.table_stride;
    const int nbk = live ? seq_blocks(context_lens, ss, a.max_blocks) : 0;
#pragma unroll
    for (int r = 0; r < BPU; ++r) {
      const int bk = b * BPU + r < nbk ? b * BPU + r : b * BPU;
      btw[r] = live ? (row[bk >> a.bs_shift] << a.bs_shift) | (bk & ((1 << a.bs_shift) - 1)) : 0;
    }
    if constexpr (ROPE) {
      pwin = live ? positions[ss] : 0;
      const int slot = live ? slot_mapping[ss] : -1;
      const int p = (live ? context_lens[ss] : 0) - 1;  // the new token's position
      rwin = -1;
      if (b == nb - 1 && slot >= 0 && p >= 0 && p < a.max_blocks * kBS) {
        // p's sub-block is the unit's sub-block r (its last with tokens); btw[r] * 16 is the slot
        // of that sub-block's first token.
        const int r = (p >> 4) - b * BPU;
        int ent = btw[0];
#pragma unroll
        for (int q = 1; q < BPU; ++q) ent = r == q ? btw[q] : ent;
        if (ent * kBS + (p & (kBS - 1)) == slot) rwin = slot;
      }
    }
  };
  // ldi: index of the unit cursor c points at.  A window refill (every 64 units) waits for
  // everything in flight once.
  // rp (ROPE): the unit's rwin entry, carried to its computation with its ring slot.
  auto load_unit = [&](const Cursor& c, int64_t ldi, uint4 (&kk)[BPU * NK], uint4 (&vv)[BPU * NV], const Tile& t,
                       int& rp) __attribute__((always_inline)) {
    if (ldi - wbase >= 64) {
      wbase = ldi;
      fill_window(c, ldi);
      __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);  // vmcnt(0)
    }
    if constexpr (ROPE) rp = __builtin_amdgcn_readlane(rwin, (int)(ldi - wbase));
    const int64_t head = (int64_t)c.kvh * (kBS << a.bs_shift) * D;
    auto off = [&](int e) __attribute__((always_inline)) {
      return (int64_t)(e >> a.bs_shift) * a.kv_stride + head + (int64_t)(e & ((1 << a.bs_shift) - 1)) * (kBS * D);
    };
    [&]<int... R>(std::integer_sequence<int, R...>) __attribute__((always_inline)) {
      ((t.template load_part<BPU, R>(kc + off(__builtin_amdgcn_readlane(btw[R], (int)(ldi - wbase))),
                                     vc + off(__builtin_amdgcn_readlane(btw[R], (int)(ldi - wbase))), kk, vv)),
       ...);
    }(std::make_integer_sequence<int, BPU>{});
  };

  Tile tile;
  tile.init(lane);
  const int H = a.num_heads;
  // Fused RoPE state (ROPE).  A segment's start loads its q rows' rotation pairs (QP per lane,
  // the G heads' D/2 pairs spread over the lanes) with their cos / sin, and the worker holding
  // the segment's last unit (kRopeHaveK) the new k row's pairs (KP per lane) and this lane's V
  // piece of the new v row.  They are rotated in the segment's first unit once that unit's next
  // loads are out (the rotation's wait then retires only loads issued before them), into
  // rope_lds (q rows [G, D], then the k row [D]); qa reads q back in the MFMA layout, the last
  // unit reads k.  rpatch[slot]: the rwin entry of the unit in that ring slot (>= 0: write the new
  // row there and put it into the loaded copy).  The segment start reads the position from the
  // window (unit j + 1 is in it when j ends, with one unit ahead).
  // Pairs per lane: G D / 128 rounded up to a power of two (runs then never cross a head's D/2
  // pairs), the lanes past the G D / 2 pairs idle.
  constexpr int QP = G * D <= 128 ? 1 : G * D <= 256 ? 2 : G * D <= 512 ? 4 : 8;
  constexpr int KP = D / 2 >= 64 ? D / 128 : 1;
  constexpr int kRopePending = 1, kRopeHaveK = 2;
  static_assert(!ROPE || kSkPrefetch == 1, "the window holds the next segment's first unit with one unit ahead");
  __shared__ __attribute__((aligned(16))) uint16_t rope_lds[ROPE ? G * D + D : 1];
  uint16_t* const rq_lds = rope_lds;
  uint16_t* const rk_lds = rope_lds + G * D;
  const int rq_p0 = lane * QP;  // this lane's first q pair over the G heads' G D/2
  const int rk_p0 = lane * KP;  // and k pair over D/2
  RopeRun<T, QP> rq;
  RopeRun<T, KP> rk;
  uint4 vnew = make_uint4(0, 0, 0, 0);
  int rope_flags = 0;
  int rpatch[NBUF];
  // Segment start at global unit ubeg + c.b.  The worker holding a segment's first block
  // (b == 0) is the first of the segment's workers: it records them for the merge kernel.
  auto begin_segment = [&](const Cursor& c, int64_t ubeg) __attribute__((always_inline)) {
    if constexpr (ROPE) {
      using S = typename Tile::S;
      const int pos = __builtin_amdgcn_readlane(pwin, (int)(ubeg - u0 - wbase));
      const float* cs = a.cos_sin + (int64_t)pos * D;
      const S* qg = q_ptr + ((int64_t)c.s * H + (int64_t)c.kvh * G) * D;
      if (rq_p0 < G * D / 2) rq.load(qg + (rq_p0 / (D / 2)) * D, cs, rq_p0 % (D / 2), D / 2);
      rope_flags = kRopePending;
      // The segment's last unit (global index ubeg + nblk - 1 - b) is this worker's.
      if (ubeg + (c.nblk - 1 - c.b) < u1) {
        rope_flags |= kRopeHaveK;
        const int64_t row = ((int64_t)c.s * hkv + c.kvh) * D;
        if (rk_p0 < D / 2) rk.load(static_cast<const S*>(a.k_new) + row, cs, rk_p0, D / 2);
        vnew = *reinterpret_cast<const uint4*>(static_cast<const S*>(a.v_new) + row + tile.vd0);
      }
    } else {
      tile.load_q(q_ptr + ((int64_t)c.s * H + (int64_t)c.kvh * G) * D);
    }
    tile.reset();
    if (c.b == 0 && lane == 0) {
      // The worker of the segment's last unit (the last k with k C / W <= its cost).
      const int64_t z = KQ * (ubeg + c.nblk - 1) + KS * (seg + 1);
      const int64_t last = ((z + 1) * W - 1) / C;
      a.seg_desc[(int64_t)c.s * hkv + c.kvh] = make_int2((int)k, (int)(last - k + 1));
    }
  };
  auto end_segment = [&](const Cursor& c) __attribute__((always_inline)) {
    float lsum[4];
    tile.reduce(lsum);
    const int64_t g = (int64_t)c.s * hkv + c.kvh;
    const int64_t idx = k + g;
    float* pa = a.part_acc + idx * (G * D);
    if (tile.vrow == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float4* dst = reinterpret_cast<float4*>(pa + h * D + tile.vd0);
#pragma unroll
        for (int q4 = 0; q4 < Tile::ACC / 4; ++q4)
          dst[q4] = make_float4(tile.acc[h][4 * q4], tile.acc[h][4 * q4 + 1], tile.acc[h][4 * q4 + 2],
                                tile.acc[h][4 * q4 + 3]);
      }
    }
    if (tile.col == 0 && tile.seg < HG) {
      float* pm = a.part_ml + idx * (2 * G);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int h = 4 * tile.seg + r;
        if (h < G) {
          pm[2 * h] = tile.m_run[r];
          pm[2 * h + 1] = lsum[r];
        }
      }
    }
  };

  const int64_t n = u1 - u0;
  Cursor ld = cur;
  int64_t ldi = 0;
  int ctx_cur = min(context_lens[cur.s], a.max_blocks * kBS);
  fill_window(cur, 0);
  uint4 kbuf[NBUF][BPU * NK], vbuf[NBUF][BPU * NV];
  // Prologue: the first kSkPrefetch units (the last one repeated past the end of the range).
#pragma unroll
  for (int q = 0; q < kSkPrefetch; ++q) {
    load_unit(ld, ldi, kbuf[q], vbuf[q], tile, rpatch[q]);
    if (q + 1 < n) {
      advance(ld);
      ++ldi;
    }
  }
  int64_t loaded = min<int64_t>(kSkPrefetch, n);  // units whose loads have been issued
  begin_segment(cur, u0);
  // Unit j computes from ring slot j % NBUF while the loads of unit j + kSkPrefetch go to
  // slot (j + kSkPrefetch) % NBUF.  Whole rounds of NBUF units run without a bounds test, so the
  // loop has no path that skips a round's loads (such a path makes the compiler drain every
  // load in flight at the loop head); the last n % NBUF units run after it.
  auto unit = [&](int64_t j, auto qc) __attribute__((always_inline)) {
    constexpr int q = decltype(qc)::value;
    load_unit(ld, ldi, kbuf[(q + kSkPrefetch) % NBUF], vbuf[(q + kSkPrefetch) % NBUF], tile,
              rpatch[(q + kSkPrefetch) % NBUF]);
    if (loaded < n) {
      ++loaded;
      if (loaded < n) {
        advance(ld);
        ++ldi;
      }
    }
    if constexpr (ROPE) {
      if (rope_flags & kRopePending) {
        if (rq_p0 < G * D / 2) rq.rotate_to(rq_lds + (rq_p0 / (D / 2)) * D, rq_p0 % (D / 2), D / 2);
        if ((rope_flags & kRopeHaveK) && rk_p0 < D / 2) rk.rotate_to(rk_lds, rk_p0, D / 2);
        // One wave per workgroup: its LDS reads follow its writes in order.
        const uint4* qrow = reinterpret_cast<const uint4*>(rq_lds + (tile.col % G) * D + 8 * tile.seg);
#pragma unroll
        for (int i = 0; i < NK; ++i) tile.qa[i] = qrow[4 * i];
        rope_flags = 0;
      }
      const int slot = rpatch[q];
      if (slot >= 0) {
        using S = typename Tile::S;
        uint4 knew[NK];
        const uint4* krow = reinterpret_cast<const uint4*>(rk_lds + 8 * tile.seg);
#pragma unroll
        for (int i = 0; i < NK; ++i) knew[i] = krow[4 * i];
        tile.template patch<BPU>(kbuf[q], vbuf[q], ((ctx_cur - 1) >> 4) - cur.b * BPU, slot & (kBS - 1), knew, vnew);
        const int bsz = kBS << a.bs_shift;
        const int64_t row = (int64_t)(slot >> (4 + a.bs_shift)) * a.kv_stride +
                            ((int64_t)cur.kvh * bsz + (slot & (bsz - 1))) * D;
        S* kdst = const_cast<S*>(kc) + row;
        S* vdst = const_cast<S*>(vc) + row;
        if (tile.col == 0) {
#pragma unroll
          for (int i = 0; i < NK; ++i) *reinterpret_cast<uint4*>(kdst + 32 * i + 8 * tile.seg) = knew[i];
        }
        if (tile.vrow == 0) *reinterpret_cast<uint4*>(vdst + tile.vd0) = vnew;
      }
    }
    tile.template step<BPU>(kbuf[q], vbuf[q], cur.b * BPU * kBS, ctx_cur, a.scale_log2, p_lds[j & 1],
                            alpha_lds[j & 1]);
    const bool last_of_segment = cur.b + 1 == cur.nblk || j + 1 == n;
    if (last_of_segment) {
      end_segment(cur);
      if (j + 1 < n) {
        ++seg;
        advance(cur);
        begin_segment(cur, u0 + j + 1);
        ctx_cur = min(context_lens[cur.s], a.max_blocks * kBS);
      }
    } else {
      advance(cur);
    }
  };
  int64_t j0 = 0;
  for (; j0 + NBUF <= n; j0 += NBUF) {
    [&]<int... Q>(std::integer_sequence<int, Q...>) {
      (unit(j0 + Q, std::integral_constant<int, Q>{}), ...);
    }(std::make_integer_sequence<int, NBUF>{});
  }
  [&]<int... Q>(std::integer_sequence<int, Q...>) {
    ((j0 + Q < n ? unit(j0 + Q, std::integral_constant<int, Q>{}) : void()), ...);
  }(std::make_integer_sequence<int, NBUF - 1>{});
}

// One workgroup per segment (sequence, kv-head), one wave per head of the group: merges the
// partials of the segment's workers (the range its first worker recorded in seg_desc) and
// writes the G output rows.  Lane l of wave h holds dims [l*D/64, (l+1)*D/64) of head h, so each
// partial's [G, D] accumulator is read as one contiguous row by the whole workgroup; every
// lane folds the partials in order with an online rescale (loads of consecutive partials
// are independent, so they are issued ahead of the folds).
template <typename T, int D, int G>
__global__ __launch_bounds__(64 * G) void decode_stream_merge_kernel(StreamArgs a,
                                                                    const int32_t* __restrict__ context_lens) {
  using S = typename elem<T>::storage;
  constexpr int PER = D / 64;  // dims per lane
  static_assert(PER == 1 || PER == 2 || PER == 4, "head_dim 64, 128 or 256");
  const int kvh = blockIdx.x;
  const int s = blockIdx.y;
  const int h = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int hkv = a.num_kv_heads;
  S* out = static_cast<S*>(a.out) + ((int64_t)s * a.num_heads + (int64_t)kvh * G + h) * D + lane * PER;
  // The segment's workers, as the first of them recorded (their partials: first + g .. ); the
  // descriptor is loaded together with the context length (one memory round trip, not two)
  // and used only when the segment has units (a segment without any keeps a stale entry).
  const int2 dsc = a.seg_desc[(int64_t)s * hkv + kvh];
  const int ctx = context_lens[s];
  asm volatile("" ::"s"(dsc.x), "s"(dsc.y), "s"(ctx));  // both loads issued before either is waited for
  if (min(ctx, a.max_blocks * kBS) <= 0) {  // no blocks (seq_blocks == 0)
#pragma unroll
    for (int e = 0; e < PER; ++e) out[e] = 0;
    return;
  }
  const int64_t pbase = (int64_t)dsc.x + (int64_t)s * hkv + kvh;  // partial index of the first worker
  const int np = dsc.y;

  float m = -INFINITY, l = 0.f;
  float acc[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) acc[e] = 0.f;
#pragma unroll 4
  for (int q = 0; q < np; ++q) {
    const int64_t pi = pbase + q;
    const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + pi * (2 * G) + 2 * h);
    const float* pa = a.part_acc + pi * (G * D) + h * D + lane * PER;
    float v[PER];
    if constexpr (PER == 4) {
      const float4 t = *reinterpret_cast<const float4*>(pa);
      v[0] = t.x;
      v[1] = t.y;
      v[2] = t.z;
      v[3] = t.w;
    } else if constexpr (PER == 2) {
      const float2 t = *reinterpret_cast<const float2*>(pa);
      v[0] = t.x;
      v[1] = t.y;
    } else {
      v[0] = pa[0];
    }
    const float mn = fmaxf(m, ml.x);
    const float fo = exp2f(m - mn);  // 0 for the first partial (m = -inf)
    const float fq = exp2f(ml.x - mn);
    l = l * fo + ml.y * fq;
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[e] = acc[e] * fo + v[e] * fq;
    m = mn;
  }
  const float inv = l != 0.f ? 1.f / l : 1.f;
  if constexpr (PER == 2 && !std::is_same_v<T, f32_t>) {
    const uint32_t packed = (uint32_t)elem<T>::from_f32(acc[0] * inv) | ((uint32_t)elem<T>::from_f32(acc[1] * inv) << 16);
    *reinterpret_cast<uint32_t*>(out) = packed;
  } else {
#pragma unroll
    for (int e = 0; e < PER; ++e) out[e] = elem<T>::from_f32(acc[e] * inv);
  }
}

// ---------------------------------------------------------------- merge -----

struct MergeArgs {
  void* out;
  const float* exp_sums;
  const float* max_logits;
  const float* tmp_out;
  const int32_t* context_lens;
  int32_t num_heads;
  int32_t head_dim;
  int32_t num_partitions;
  int32_t partition_size;
  int32_t skip_single;  // 1: sequences with one partition were written by the partition kernel
};

// One workgroup of 256 threads per (seq, q-head).  The partition weights e^(m_p - M) go to LDS
// once per partition; thread t accumulates the float4 column chunk c = t % C of the rows
// p = g, g + R, ... of tmp_out (C = D / 4 chunks per row, g = t / C, R = 256 / C row groups),
// so R rows are read at a time, and the R partial sums are added in group order through LDS
// (a fixed order: the result does not depend on timing).
constexpr int kMergeThreads = 256;
template <typename T>
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(MergeArgs a) {
  using E = elem<T>;
  using S = typename E::storage;
  constexpr int kChunk = kMergeThreads;  // partitions whose weights sit in LDS at a time
  constexpr int kWaves = kMergeThreads / 64;
  __shared__ float w_lds[kChunk];
  __shared__ float red[2 * kWaves];
  __shared__ float4 part[kMergeThreads];
  const int h = blockIdx.x;
  const int s = blockIdx.y;
  const int tid = threadIdx.x;
  const int wv = tid >> 6;
  const int D = a.head_dim;
  const int ctx = max(0, a.context_lens[s]);
  const int np_s = min(num_parts_for(ctx, a.partition_size), a.num_partitions);
  if (a.skip_single && np_s <= 1) return;
  S* op = static_cast<S*>(a.out) + ((int64_t)s * a.num_heads + h) * D;
  if (np_s == 0) {
    for (int d = tid; d < D; d += kMergeThreads) E::store(op, d, 0.f);
    return;
  }
  const int64_t sh = ((int64_t)s * a.num_heads + h) * a.num_partitions;
  const float* ml = a.max_logits + sh;
  const float* es = a.exp_sums + sh;
  float M = -INFINITY;
  for (int q = tid; q < np_s; q += kMergeThreads) M = fmaxf(M, ml[q]);
  M = wave_max(M);
  if ((tid & 63) == 0) red[wv] = M;
  __syncthreads();
  M = red[0];
#pragma unroll
  for (int j = 1; j < kWaves; ++j) M = fmaxf(M, red[j]);
  float L = 0.f;
  for (int q = tid; q < np_s; q += kMergeThreads) L += expf(ml[q] - M) * es[q];
  L = wave_sum(L);
  if ((tid & 63) == 0) red[kWaves + wv] = L;
  __syncthreads();
  L = red[kWaves];
#pragma unroll
  for (int j = 1; j < kWaves; ++j) L += red[kWaves + j];
  const float inv = L != 0.f ? 1.f / L : 1.f;
  const float* tp = a.tmp_out + sh * D;
  const int C = D / 4;                    // head_dim % 4 == 0 and <= 1024 (checked on the host)
  const int R = kMergeThreads / C;
  const int c = tid % C, g = tid / C;
  const bool active = g < R;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int q0 = 0; q0 < np_s; q0 += kChunk) {
    const int n = min(kChunk, np_s - q0);
    __syncthreads();  // the previous chunk's weights are no longer read
    if (tid < n) w_lds[tid] = expf(ml[q0 + tid] - M);
    __syncthreads();
    if (active) {
#pragma unroll 4
      for (int q = g; q < n; q += R) {
        const float r = w_lds[q];
        const float4 v = *reinterpret_cast<const float4*>(tp + (int64_t)(q0 + q) * D + 4 * c);
        acc.x += r * v.x;
        acc.y += r * v.y;
        acc.z += r * v.z;
        acc.w += r * v.w;
      }
    }
  }
  if (active) part[g * C + c] = acc;
  __syncthreads();
  if (tid < C) {
    float4 t = part[tid];
    for (int j = 1; j < R; ++j) {
      const float4 u = part[j * C + tid];
      t.x += u.x;
      t.y += u.y;
      t.z += u.z;
      t.w += u.w;
    }
    E::store(op, 4 * tid + 0, t.x * inv);
    E::store(op, 4 * tid + 1, t.y * inv);
    E::store(op, 4 * tid + 2, t.z * inv);
    E::store(op, 4 * tid + 3, t.w * inv);
  }
}

// ------------------------------------------------------------ host side -----

// Tokens per partition the v1 entries use when given a workspace.
#ifndef RG_V1_PARTITION
#define RG_V1_PARTITION 256
#endif
constexpr int kV1PartitionTokens = RG_V1_PARTITION;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct Shape {
  int32_t H, Hkv, D, bs, MB, B;
};

int check_decode_shape(const char* op, const Shape& sh, int32_t dtype, int64_t kv_stride) {
  if (dtype_bytes(dtype) == 0) return fail(RG_ERR_NOT_SUPPORTED, "%s: unknown dtype %d", op, dtype);
  if (sh.D % 4 != 0 || sh.D > RG_MAX_HEAD_DIM || sh.D <= 0) {
    return fail(RG_ERR_NOT_SUPPORTED,
                "not supported: PagedAttention - head_dim must be a multiple of 4 and <= %d, "
                "but got %d", RG_MAX_HEAD_DIM, sh.D);
  }
  if (sh.B < 0 || sh.H <= 0 || sh.Hkv <= 0 || sh.bs <= 0 || sh.MB < 0) {
    return fail(RG_ERR_INVALID_ARGUMENT,
                "%s: need batch >= 0, max_blocks_per_seq >= 0 and positive heads/block_size", op);
  }
  if (sh.H % sh.Hkv != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: num_heads %d is not a multiple of num_kv_heads %d",
                op, sh.H, sh.Hkv);
  }
  if (kv_stride != 0 && kv_stride < (int64_t)sh.Hkv * sh.bs * sh.D) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: kv_block_stride %lld smaller than a block", op,
                (long long)kv_stride);
  }
  return RG_OK;
}

template <typename T, int D, int G>
void launch_mfma(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((decode_mfma_kernel<T, D, G>), grid, dim3(kThreads), 0, s, a,
                     static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.k_cache),
                     static_cast<const uint16_t*>(a.v_cache), a.block_table, a.context_lens);
}

template <typename T, int D>
bool launch_mfma_g(const DecodeArgs& a, int G, dim3 grid, hipStream_t s) {
  switch (G) {
    case 1: launch_mfma<T, D, 1>(a, grid, s); return true;
    case 2: launch_mfma<T, D, 2>(a, grid, s); return true;
    case 4: launch_mfma<T, D, 4>(a, grid, s); return true;
    case 8: launch_mfma<T, D, 8>(a, grid, s); return true;
    case 3:
    case 5:
    case 6:
    case 7:
      if constexpr (D <= 128) {
        if (G == 3) launch_mfma<T, D, 3>(a, grid, s);
        else if (G == 5) launch_mfma<T, D, 5>(a, grid, s);
        else if (G == 6) launch_mfma<T, D, 6>(a, grid, s);
        else launch_mfma<T, D, 7>(a, grid, s);
        return true;
      }
      return false;
    case 16:
      if constexpr (D < 256) {
        launch_mfma<T, D, 16>(a, grid, s);
        return true;
      }
      return false;
    default: return false;
  }
}

// GQA ratios of the MFMA tiles: the q-heads of a kv-head are replicated over the 16 rows of the
// A operand (row m holds head m % G), so any G up to 16 has its heads in the first G rows; the
// powers of two at every head_dim, G = 3, 5, 6 and 7 (Llama-3.2-3B 24/8, Qwen2.5-14B 40/8,
// Qwen2-7B 28/4, ...) at head_dim 64 and 128.
bool mfma_group_size(int G, int head_dim) {
  return G == 1 || G == 2 || G == 4 || G == 8 || G == 16 ||
         ((G == 3 || G == 5 || G == 6 || G == 7) && head_dim <= 128);
}

bool mfma_applies(const DecodeArgs& a, int32_t dtype) {
  const int G = a.num_heads / a.num_kv_heads;
  const int eb = dtype_bytes(dtype);
  return (dtype == RG_DTYPE_BF16 || dtype == RG_DTYPE_F16) && a.bs_shift >= 0 &&
         (a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256) &&
         mfma_group_size(G, a.head_dim) && a.partition_size % kBS == 0 &&
         aligned16(a.q) && aligned16(a.k_cache) && aligned16(a.v_cache) &&
         (a.kv_stride * eb) % 16 == 0 &&
         (a.out == nullptr || (reinterpret_cast<uintptr_t>(a.out) & 3u) == 0);
}

// The grid kernel: the MFMA shapes but head_dim 256 with 16 q-heads per kv-head (whose
// accumulators and two K/V blocks in flight exceed the registers of a wave).
bool grid_mfma_applies(const DecodeArgs& a, int32_t dtype) {
  return mfma_applies(a, dtype) && !(a.head_dim == 256 && a.num_heads / a.num_kv_heads == 16);
}

// The stream-K decode: the MFMA shapes in bf16 / f16, and the same shapes in fp32 (head_dim 64,
// 128 or 256; at 256 a worker holds a block's K and V rows, 128 VGPRs, next to the q row's 64: it
// runs with AGPRs as extra registers, one wave per SIMD as always).
bool stream_applies(const DecodeArgs& a, int32_t dtype) {
  if (dtype != RG_DTYPE_F32) return mfma_applies(a, dtype);
  const int G = a.num_heads / a.num_kv_heads;
  return a.bs_shift >= 0 && (a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256) &&
         mfma_group_size(G, a.head_dim) && aligned16(a.q) && aligned16(a.k_cache) &&
         aligned16(a.v_cache) && (a.kv_stride * 4) % 16 == 0 && (a.out == nullptr || (reinterpret_cast<uintptr_t>(a.out) & 3u) == 0);
}

// Launches the partition kernel over grid (grid_parts, heads, batch).
int run_partition(const char* op, const DecodeArgs& a, int32_t dtype, int32_t batch,
                  int32_t grid_parts, hipStream_t s) {
  if (batch == 0 || grid_parts == 0) return ok();
  if (grid_mfma_applies(a, dtype)) {
    const int G = a.num_heads / a.num_kv_heads;
    const dim3 grid(grid_parts, a.num_kv_heads, batch);
    if (dtype == RG_DTYPE_BF16) {
      if (a.head_dim == 256) launch_mfma_g<bf16_t, 256>(a, G, grid, s);
      else if (a.head_dim == 128) launch_mfma_g<bf16_t, 128>(a, G, grid, s);
      else launch_mfma_g<bf16_t, 64>(a, G, grid, s);
    } else {
      if (a.head_dim == 256) launch_mfma_g<f16_t, 256>(a, G, grid, s);
      else if (a.head_dim == 128) launch_mfma_g<f16_t, 128>(a, G, grid, s);
      else launch_mfma_g<f16_t, 64>(a, G, grid, s);
    }
    return check_launch(op);
  }
  const dim3 grid(grid_parts, a.num_heads, batch);
  return dispatch_dtype(dtype, [&](auto tag) {
    hipLaunchKernelGGL(decode_generic_kernel<decltype(tag)>, grid, dim3(64), 0, s, a);
    return check_launch(op);
  });
}

int run_merge(const char* op, const MergeArgs& m, int32_t dtype, int32_t batch, hipStream_t s) {
  if (batch == 0) return ok();
  const dim3 grid(m.num_heads, batch);
  return dispatch_dtype(dtype, [&](auto tag) {
    hipLaunchKernelGGL(decode_merge_kernel<decltype(tag)>, grid, dim3(kMergeThreads), 0, s, m);
    return check_launch(op);
  });
}

DecodeArgs make_args(const void* q, const void* kc, const void* vc, const int32_t* bt,
                     const int32_t* cl, void* out, float scale, const Shape& sh,
                     int64_t kv_stride, int32_t P, int32_t NP, int32_t mode) {
  DecodeArgs a;
  a.q = q;
  a.k_cache = kc;
  a.v_cache = vc;
  a.block_table = bt;
  a.context_lens = cl;
  a.out = out;
  a.tmp_out = nullptr;
  a.exp_sums = nullptr;
  a.max_logits = nullptr;
  a.scale_log2 = scale * kLog2e;
  a.num_heads = sh.H;
  a.num_kv_heads = sh.Hkv;
  a.head_dim = sh.D;
  a.block_size = sh.bs;
  a.max_blocks = sh.MB;
  a.num_partitions = NP;
  a.partition_size = P;
  a.kv_stride = kv_stride ? kv_stride : (int64_t)sh.Hkv * sh.bs * sh.D;
  a.mode = mode;
  a.bs_shift = -1;
  for (int j = 0; j <= 4; ++j)
    if (sh.bs == (kBS << j)) a.bs_shift = j;
  return a;
}

struct V2Scratch {
  float* tmp_out;
  float* exp_sums;
  float* max_logits;
};

size_t v2_bytes(int64_t B, int64_t H, int64_t NP, int64_t D, V2Scratch* carve, void* base) {
  const size_t n_stat = (size_t)(B * H * NP);
  const size_t tmp = align_up(n_stat * (size_t)D * 4, 256);
  const size_t stat = align_up(n_stat * 4, 256);
  if (carve) {
    char* p = static_cast<char*>(base);
    carve->tmp_out = reinterpret_cast<float*>(p);
    carve->exp_sums = reinterpret_cast<float*>(p + tmp);
    carve->max_logits = reinterpret_cast<float*>(p + tmp + stat);
  }
  return tmp + 2 * stat;
}

int32_t v1_num_partitions(const Shape& sh) {
  const int64_t max_ctx = (int64_t)sh.MB * sh.bs;
  return (int32_t)ceil_div(max_ctx, kV1PartitionTokens);
}

// ---- stream-K path ----

// Waves per CU the stream-K decode launches (one worker per wave).
#ifndef RG_SK_WAVES_PER_CU
#define RG_SK_WAVES_PER_CU 4
#endif

int32_t stream_workers(const Shape& sh) {
  const int64_t want = (int64_t)device_cu_count() * RG_SK_WAVES_PER_CU;
  const int64_t units_max = (int64_t)sh.B * sh.Hkv * std::max(sh.MB, 1) * std::max(sh.bs / kBS, 1);
  return (int32_t)std::max<int64_t>(1, std::min(want, units_max));
}

struct StreamScratch {
  float* acc;
  float* ml;
  int2* desc;
};

size_t stream_bytes(const Shape& sh, int32_t workers, StreamScratch* carve, void* base) {
  const int64_t G = sh.H / sh.Hkv;
  const int64_t segments = (int64_t)sh.B * sh.Hkv;
  const int64_t partials = (int64_t)workers + segments;
  const size_t acc = align_up((size_t)(partials * G * sh.D) * 4, 256);
  const size_t ml = align_up((size_t)(partials * G * 2) * 4, 256);
  const size_t desc = align_up((size_t)segments * sizeof(int2), 256);
  if (carve) {
    carve->acc = static_cast<float*>(base);
    carve->ml = reinterpret_cast<float*>(static_cast<char*>(base) + acc);
    carve->desc = reinterpret_cast<int2*>(static_cast<char*>(base) + acc + ml);
  }
  return acc + ml + desc;
}

template <typename T, int D, int G, bool ROPE = false>
void launch_stream(const StreamArgs& sa, const DecodeArgs& a, hipStream_t s) {
  using S = typename DecodeTileFor<T, D, G>::S;
  hipLaunchKernelGGL((decode_stream_kernel<T, D, G, ROPE>), dim3(sa.num_workers), dim3(64), 0, s, sa,
                     static_cast<const S*>(a.q), static_cast<const S*>(a.k_cache),
                     static_cast<const S*>(a.v_cache), a.block_table, a.context_lens, sa.positions,
                     sa.slot_mapping);
  hipLaunchKernelGGL((decode_stream_merge_kernel<T, D, G>), dim3(sa.num_kv_heads, sa.batch), dim3(64 * G), 0, s,
                     sa, a.context_lens);
}

template <typename T, int D>
void launch_stream_g(const StreamArgs& sa, const DecodeArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: launch_stream<T, D, 1>(sa, a, s); break;
    case 2: launch_stream<T, D, 2>(sa, a, s); break;
    case 4: launch_stream<T, D, 4>(sa, a, s); break;
    case 8: launch_stream<T, D, 8>(sa, a, s); break;
    case 16: launch_stream<T, D, 16>(sa, a, s); break;
    default:
      // G = 3, 5, 6, 7 (stream_applies admits them at head_dim 64 and 128 only)
      if constexpr (D <= 128) {
        if (G == 3) launch_stream<T, D, 3>(sa, a, s);
        else if (G == 5) launch_stream<T, D, 5>(sa, a, s);
        else if (G == 6) launch_stream<T, D, 6>(sa, a, s);
        else if (G == 7) launch_stream<T, D, 7>(sa, a, s);
      }
      break;
  }
}

// The step's new tokens for the fused RoPE form: rows [batch, H_kv, D] of k and v, token s
// being sequence s's.
struct RopeIn {
  const void* k;
  const void* v;
  const float* cos_sin;
  const int32_t* positions;
  const int32_t* slot_mapping;
};

// The fused RoPE form runs at bf16 / f16, head_dim 64 and 128 and G 1 to 8.
bool rope_stream_applies(const DecodeArgs& a, int32_t dtype, const RopeIn& r) {
  const int G = a.num_heads / a.num_kv_heads;
  return (dtype == RG_DTYPE_BF16 || dtype == RG_DTYPE_F16) && stream_applies(a, dtype) &&
         (a.head_dim == 64 || a.head_dim == 128) && G >= 1 && G <= 8 && aligned16(r.k) && aligned16(r.v) &&
         aligned16(r.cos_sin);
}

template <typename T, int D>
void launch_stream_rope_g(const StreamArgs& sa, const DecodeArgs& a, int G, hipStream_t s) {
  switch (G) {
    case 1: launch_stream<T, D, 1, true>(sa, a, s); break;
    case 2: launch_stream<T, D, 2, true>(sa, a, s); break;
    case 3: launch_stream<T, D, 3, true>(sa, a, s); break;
    case 4: launch_stream<T, D, 4, true>(sa, a, s); break;
    case 5: launch_stream<T, D, 5, true>(sa, a, s); break;
    case 6: launch_stream<T, D, 6, true>(sa, a, s); break;
    case 7: launch_stream<T, D, 7, true>(sa, a, s); break;
    default: launch_stream<T, D, 8, true>(sa, a, s); break;  // G = 8 (rope_stream_applies)
  }
}

// Runs the stream-K decode if it applies and the workspace holds its scratch; returns
// RG_ERR_WORKSPACE (without recording an error) when the workspace is too small.  With rope,
// the fused RoPE form (rope_stream_applies holds).
int run_stream(const char* op, const DecodeArgs& a, int32_t dtype, const Shape& sh, void* ws, size_t ws_bytes,
               hipStream_t s, const RopeIn* rope = nullptr) {
  const int32_t workers = stream_workers(sh);
  StreamScratch sc;
  if (ws_bytes < stream_bytes(sh, workers, &sc, ws)) return RG_ERR_WORKSPACE;
  StreamArgs sa{};
  sa.out = a.out;
  sa.part_acc = sc.acc;
  sa.part_ml = sc.ml;
  sa.seg_desc = sc.desc;
  sa.scale_log2 = a.scale_log2;
  sa.num_heads = sh.H;
  sa.num_kv_heads = sh.Hkv;
  sa.max_blocks = sh.MB << a.bs_shift;
  sa.batch = sh.B;
  sa.num_workers = workers;
  sa.kv_stride = a.kv_stride;
  sa.table_stride = sh.MB;
  sa.bs_shift = a.bs_shift;
  const int G = sh.H / sh.Hkv;
  if (rope != nullptr) {
    sa.k_new = rope->k;
    sa.v_new = rope->v;
    sa.cos_sin = rope->cos_sin;
    sa.positions = rope->positions;
    sa.slot_mapping = rope->slot_mapping;
    if (dtype == RG_DTYPE_BF16) {
      if (sh.D == 128) launch_stream_rope_g<bf16_t, 128>(sa, a, G, s);
      else launch_stream_rope_g<bf16_t, 64>(sa, a, G, s);
    } else {
      if (sh.D == 128) launch_stream_rope_g<f16_t, 128>(sa, a, G, s);
      else launch_stream_rope_g<f16_t, 64>(sa, a, G, s);
    }
    return check_launch(op);
  }
  if (dtype == RG_DTYPE_BF16) {
    if (sh.D == 256) launch_stream_g<bf16_t, 256>(sa, a, G, s);
    else if (sh.D == 128) launch_stream_g<bf16_t, 128>(sa, a, G, s);
    else launch_stream_g<bf16_t, 64>(sa, a, G, s);
  } else if (dtype == RG_DTYPE_F16) {
    if (sh.D == 256) launch_stream_g<f16_t, 256>(sa, a, G, s);
    else if (sh.D == 128) launch_stream_g<f16_t, 128>(sa, a, G, s);
    else launch_stream_g<f16_t, 64>(sa, a, G, s);
  } else {
    if (sh.D == 256) launch_stream_g<f32_t, 256>(sa, a, G, s);
    else if (sh.D == 128) launch_stream_g<f32_t, 128>(sa, a, G, s);
    else launch_stream_g<f32_t, 64>(sa, a, G, s);
  }
  return check_launch(op);
}

// Body shared by the v1 and v1_plus entries.
int paged_v1(const char* op, const void* q, const void* kc, const void* vc, const int32_t* bt,
             const int32_t* cl, void* out, float scale, const Shape& sh, int32_t dtype,
             int64_t kv_stride, void* ws, size_t ws_bytes, void* stream) {
  int st = check_decode_shape(op, sh, dtype, kv_stride);
  if (st != RG_OK) return st;
  if (sh.B == 0) return ok();
  if (!q || !kc || !vc || !bt || !cl || !out) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  hipStream_t s = as_stream(stream);
  if (ws != nullptr) {
    DecodeArgs a = make_args(q, kc, vc, bt, cl, out, scale, sh, kv_stride, kBS, 1, MODE_AUTO);
    if (stream_applies(a, dtype) && sh.MB > 0) {
      st = run_stream(op, a, dtype, sh, ws, ws_bytes, s);
      if (st != RG_ERR_WORKSPACE) return st;
      return fail(RG_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu required", op, ws_bytes,
                  stream_bytes(sh, stream_workers(sh), nullptr, nullptr));
    }
  }
  const int32_t np = v1_num_partitions(sh);
  if (ws != nullptr && np > 1) {
    V2Scratch sc;
    const size_t need = v2_bytes(sh.B, sh.H, np, sh.D, &sc, ws);
    if (ws_bytes < need) {
      return fail(RG_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu required", op, ws_bytes, need);
    }
    DecodeArgs a = make_args(q, kc, vc, bt, cl, out, scale, sh, kv_stride, kV1PartitionTokens, np,
                             MODE_AUTO);
    a.tmp_out = sc.tmp_out;
    a.exp_sums = sc.exp_sums;
    a.max_logits = sc.max_logits;
    st = run_partition(op, a, dtype, sh.B, np, s);
    if (st != RG_OK) return st;
    MergeArgs m{out, sc.exp_sums, sc.max_logits, sc.tmp_out, cl, sh.H, sh.D, np,
                kV1PartitionTokens, 1};
    return run_merge(op, m, dtype, sh.B, s);
  }
  // One partition spans the whole block table.
  const int32_t P = (int32_t)std::max<int64_t>(16, ceil_div((int64_t)sh.MB * sh.bs, 16) * 16);
  DecodeArgs a = make_args(q, kc, vc, bt, cl, out, scale, sh, kv_stride, P, 1, MODE_FINAL);
  return run_partition(op, a, dtype, sh.B, 1, s);
}

// ---- entry without allocation ----
//
// rg_paged_attention_v1_no_alloc keeps the stream-K partials in `scratch` below, one copy per
// device, instead of a caller's workspace.  Host code never passes `scratch` itself to a
// kernel (on the host that name is a stand-in, not a device address): the address of each
// device's copy comes from hipGetSymbolAddress, taken once per device with that device
// current, and is kept in g_scratch_addr.

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

}  // namespace

static __device__ __align__(256) unsigned char scratch[RG_NO_ALLOC_SCRATCH_BYTES];

namespace {

// Address of the current device's copy of `scratch`; looked up on the first call per device.
int no_alloc_scratch(const char* op, void** addr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(RG_ERR_HIP, "%s: no current device: %s", op, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) {
    return fail(RG_ERR_NOT_SUPPORTED, "%s: device ordinal %d beyond the %d devices supported", op, dev, kMaxDevices);
  }
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr) {
        return fail(RG_ERR_HIP, "%s: cannot locate the static scratch on device %d: %s", op, dev,
                    hipGetErrorString(e));
      }
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return RG_OK;
}

}  // namespace

// Called by rg_init with the device being initialised current.
int setup_no_alloc_scratch() {
  void* p = nullptr;
  return no_alloc_scratch("rg_init", &p);
}

int probe_decode_kernels() {
  hipFuncAttributes at;
  if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(decode_mfma_kernel<bf16_t, 128, 4>)) !=
          hipSuccess ||
      hipFuncGetAttributes(&at, reinterpret_cast<const void*>(decode_generic_kernel<f32_t>)) !=
          hipSuccess) {
    return fail(RG_ERR_HIP, "failed to load the decode kernels: %s",
                hipGetErrorString(hipGetLastError()));
  }
  return RG_OK;
}

}  // namespace rg

using namespace rg;

extern "C" size_t rg_paged_attention_v1_workspace_bytes(int32_t batch_size, int32_t num_heads,
                                                        int32_t num_kv_heads, int32_t head_dim,
                                                        int32_t block_size, int32_t max_blocks_per_seq) {
  if (batch_size <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      head_dim <= 0 || block_size <= 0 || max_blocks_per_seq <= 0) {
    return 0;
  }
  const Shape sh{num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size};
  const int32_t np = v1_num_partitions(sh);
  const size_t grid = np > 1 ? v2_bytes(batch_size, num_heads, np, head_dim, nullptr, nullptr) : 0;
  return std::max(grid, stream_bytes(sh, stream_workers(sh), nullptr, nullptr));
}

extern "C" int rg_paged_attention_v1(const void* query, const void* key_cache,
                                     const void* value_cache, const int32_t* block_table,
                                     const int32_t* context_lens, void* output, float scale,
                                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t block_size, int32_t max_blocks_per_seq,
                                     int32_t batch_size, int32_t dtype, int64_t kv_block_stride,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  const Shape sh{num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size};
  return paged_v1("paged_attention_v1", query, key_cache, value_cache, block_table, context_lens,
                  output, scale, sh, dtype, kv_block_stride, workspace, workspace_bytes, stream);
}

extern "C" int rg_rope_reshape_and_cache_paged_attention_v1(
    const void* query, const void* key, const void* value, void* key_cache, void* value_cache,
    const float* cos_sin, const int32_t* positions, const int32_t* slot_mapping, const int32_t* block_table,
    const int32_t* context_lens, void* output, float scale, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq, int32_t batch_size, int32_t dtype,
    int64_t kv_block_stride, void* workspace, size_t workspace_bytes, void* stream) {
  const char* op = "rope_reshape_and_cache_paged_attention_v1";
  const Shape sh{num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size};
  int st = check_decode_shape(op, sh, dtype, kv_block_stride);
  if (st != RG_OK) return st;
  if (sh.B == 0) return ok();
  if (!query || !key || !value || !key_cache || !value_cache || !cos_sin || !positions || !slot_mapping ||
      !block_table || !context_lens || !output) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  if (workspace == nullptr) return fail(RG_ERR_INVALID_ARGUMENT, "%s: needs a workspace", op);
  const DecodeArgs a = make_args(query, key_cache, value_cache, block_table, context_lens, output, scale, sh,
                                 kv_block_stride, kBS, 1, MODE_AUTO);
  const RopeIn rope{key, value, cos_sin, positions, slot_mapping};
  if (sh.MB <= 0 || !rope_stream_applies(a, dtype, rope)) {
    return fail(RG_ERR_NOT_SUPPORTED,
                "%s: runs at bf16 / f16, head_dim 64 or 128, num_heads / num_kv_heads 1 to 8, "
                "block_size 16 * 2^j and 16-byte aligned rows (rg_rope_reshape_and_cache followed by "
                "rg_paged_attention_v1 covers the rest)", op);
  }
  st = run_stream(op, a, dtype, sh, workspace, workspace_bytes, as_stream(stream), &rope);
  if (st != RG_ERR_WORKSPACE) return st;
  return fail(RG_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu required", op, workspace_bytes,
              stream_bytes(sh, stream_workers(sh), nullptr, nullptr));
}

extern "C" int rg_paged_attention_v1_plus(const void* query, const void* key_cache,
                                          const void* value_cache, const int32_t* block_table,
                                          const int32_t* context_lens, void* output,
                                          const float* rotation_metadata, float scale,
                                          int32_t num_heads, int32_t num_kv_heads,
                                          int32_t head_dim, int32_t block_size,
                                          int32_t max_blocks_per_seq, int32_t batch_size,
                                          int32_t dtype, int64_t kv_block_stride, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  (void)rotation_metadata;  // identity rotation
  const Shape sh{num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size};
  return paged_v1("paged_attention_v1_plus", query, key_cache, value_cache, block_table,
                  context_lens, output, scale, sh, dtype, kv_block_stride, workspace,
                  workspace_bytes, stream);
}

extern "C" size_t rg_v2_workspace_bytes(int32_t batch_size, int32_t num_heads,
                                        int32_t num_partitions, int32_t head_dim) {
  if (batch_size <= 0 || num_heads <= 0 || num_partitions <= 0 || head_dim <= 0) return 0;
  return v2_bytes(batch_size, num_heads, num_partitions, head_dim, nullptr, nullptr);
}

extern "C" int rg_paged_attention_v2_partition(
    const void* query, const void* key_cache, const void* value_cache, const int32_t* block_table,
    const int32_t* context_lens, float* tmp_out, float* exp_sums, float* max_logits,
    const float* rotation_metadata, float scale, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq, int32_t num_partitions,
    int32_t batch_size, int32_t partition_size, int32_t dtype, int64_t kv_block_stride,
    void* stream) {
  (void)rotation_metadata;
  const char* op = "paged_attention_v2_partition";
  const Shape sh{num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size};
  int st = check_decode_shape(op, sh, dtype, kv_block_stride);
  if (st != RG_OK) return st;
  if (partition_size <= 0 || partition_size % block_size != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT,
                "%s: partition_size %d must be a positive multiple of block_size %d", op,
                partition_size, block_size);
  }
  if (num_partitions < 0) return fail(RG_ERR_INVALID_ARGUMENT, "%s: num_partitions < 0", op);
  if (batch_size == 0 || num_partitions == 0) return ok();
  if (!query || !key_cache || !value_cache || !block_table || !context_lens || !tmp_out ||
      !exp_sums || !max_logits) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  DecodeArgs a = make_args(query, key_cache, value_cache, block_table, context_lens, nullptr,
                           scale, sh, kv_block_stride, partition_size, num_partitions,
                           MODE_PARTIAL);
  a.tmp_out = tmp_out;
  a.exp_sums = exp_sums;
  a.max_logits = max_logits;
  return run_partition(op, a, dtype, batch_size, num_partitions, as_stream(stream));
}

extern "C" int rg_paged_attention_v2_reduce(void* output, const float* exp_sums,
                                            const float* max_logits, const float* tmp_out,
                                            const int32_t* context_lens,
                                            const float* rotation_metadata, int32_t num_heads,
                                            int32_t head_dim, int32_t num_partitions,
                                            int32_t batch_size, int32_t partition_size,
                                            int32_t dtype, void* stream) {
  (void)rotation_metadata;
  const char* op = "paged_attention_v2_reduce";
  if (dtype_bytes(dtype) == 0) return fail(RG_ERR_NOT_SUPPORTED, "%s: unknown dtype %d", op, dtype);
  if (head_dim > 1024) {
    // MAX_HEAD_DIM_V2_REDUCE (crates/vllm-cuda/src/kernels/mod.rs:477-482)
    return fail(RG_ERR_INVALID_ARGUMENT,
                "head_dim %d exceeds maximum block size 1024 for reduction kernel", head_dim);
  }
  if (head_dim <= 0 || head_dim % 4 != 0) {
    return fail(RG_ERR_NOT_SUPPORTED, "%s: head_dim must be a positive multiple of 4, got %d", op,
                head_dim);
  }
  if (num_heads <= 0 || batch_size < 0 || num_partitions < 0 || partition_size <= 0) {
    return fail(RG_ERR_INVALID_ARGUMENT,
                "%s: need num_heads > 0, batch >= 0, num_partitions >= 0, partition_size > 0",
                op);
  }
  if (batch_size == 0) return ok();
  if (!output || !context_lens || (num_partitions > 0 && (!exp_sums || !max_logits || !tmp_out))) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  MergeArgs m{output, exp_sums, max_logits, tmp_out, context_lens, num_heads, head_dim,
              num_partitions, partition_size, 0};
  return run_merge(op, m, dtype, batch_size, as_stream(stream));
}

extern "C" int rg_paged_attention_v2(const void* query, const void* key_cache,
                                     const void* value_cache, const int32_t* block_table,
                                     const int32_t* context_lens, void* output, float scale,
                                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t block_size, int32_t max_blocks_per_seq,
                                     int32_t batch_size, int32_t max_context_len,
                                     int32_t partition_size, int32_t dtype,
                                     int64_t kv_block_stride, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  const char* op = "paged_attention_v2";
  const Shape sh{num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size};
  int st = check_decode_shape(op, sh, dtype, kv_block_stride);
  if (st != RG_OK) return st;
  if (partition_size <= 0 || partition_size % block_size != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT,
                "%s: partition_size %d must be a positive multiple of block_size %d", op,
                partition_size, block_size);
  }
  if (max_context_len < 0) return fail(RG_ERR_INVALID_ARGUMENT, "%s: max_context_len < 0", op);
  if (batch_size == 0) return ok();
  if (!query || !key_cache || !value_cache || !block_table || !context_lens || !output) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  hipStream_t s = as_stream(stream);
  if (workspace != nullptr) {
    // The stream-K decode computes the same merge of split-K partials with balanced splits;
    // it runs whenever it applies and the workspace holds its scratch.
    DecodeArgs a = make_args(query, key_cache, value_cache, block_table, context_lens, output, scale, sh,
                             kv_block_stride, partition_size, 1, MODE_AUTO);
    if (stream_applies(a, dtype) && max_blocks_per_seq > 0) {
      st = run_stream(op, a, dtype, sh, workspace, workspace_bytes, s);
      if (st != RG_ERR_WORKSPACE) return st;
    }
  }
  const int32_t np = (int32_t)std::max<int64_t>(1, ceil_div(max_context_len, partition_size));
  V2Scratch sc;
  const size_t need = v2_bytes(batch_size, num_heads, np, head_dim, &sc, workspace);
  if (workspace == nullptr || workspace_bytes < need) {
    return fail(RG_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu required", op,
                workspace ? workspace_bytes : (size_t)0, need);
  }
  DecodeArgs a = make_args(query, key_cache, value_cache, block_table, context_lens, output, scale,
                           sh, kv_block_stride, partition_size, np, MODE_AUTO);
  a.tmp_out = sc.tmp_out;
  a.exp_sums = sc.exp_sums;
  a.max_logits = sc.max_logits;
  st = run_partition(op, a, dtype, batch_size, np, s);
  if (st != RG_OK) return st;
  MergeArgs m{output, sc.exp_sums, sc.max_logits, sc.tmp_out, context_lens, num_heads, head_dim,
              np, partition_size, 1};
  return run_merge(op, m, dtype, batch_size, s);
}

extern "C" int rg_paged_attention_v1_no_alloc(const void* query, const void* key_cache,
                                              const void* value_cache, const int32_t* block_table,
                                              const int32_t* context_lens, void* output, float scale,
                                              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                              int32_t block_size, int32_t max_blocks_per_seq,
                                              int32_t batch_size, int32_t dtype, int64_t kv_block_stride,
                                              void* stream) {
  const char* op = "paged_attention_v1_no_alloc";
  const Shape sh{num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, batch_size};
  int st = check_decode_shape(op, sh, dtype, kv_block_stride);
  if (st != RG_OK) return st;
  if (sh.B == 0) return ok();
  if (!query || !key_cache || !value_cache || !block_table || !context_lens || !output) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  const DecodeArgs a = make_args(query, key_cache, value_cache, block_table, context_lens, output, scale, sh,
                                 kv_block_stride, kBS, 1, MODE_AUTO);
  if (stream_applies(a, dtype) && sh.MB > 0) {
    // The stream-K kernels of rg_paged_attention_v1 with the static scratch as their workspace.
    // Nothing in it needs clearing: every partial and segment descriptor the merge reads is
    // written earlier in the same call.
    const size_t need = stream_bytes(sh, stream_workers(sh), nullptr, nullptr);
    if (need > (size_t)RG_NO_ALLOC_SCRATCH_BYTES) {
      return fail(RG_ERR_WORKSPACE,
                  "%s: this shape needs %zu bytes of split-K scratch, the static scratch holds %zu "
                  "(call rg_paged_attention_v1 with a workspace instead)",
                  op, need, (size_t)RG_NO_ALLOC_SCRATCH_BYTES);
    }
    void* ws = nullptr;
    st = no_alloc_scratch(op, &ws);
    if (st != RG_OK) return st;
    return run_stream(op, a, dtype, sh, ws, RG_NO_ALLOC_SCRATCH_BYTES, as_stream(stream));
  }
  // The other paths of rg_paged_attention_v1 without a workspace use no scratch at all.
  return paged_v1(op, query, key_cache, value_cache, block_table, context_lens, output, scale, sh, dtype,
                  kv_block_stride, nullptr, 0, stream);
}
