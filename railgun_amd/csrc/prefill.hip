// Packed causal prefill over a paged KV cache.
//
// Sequence s owns query rows [cu_seqlens[s], cu_seqlens[s+1]) of the packed
// stream; its context of context_lens[s] tokens (earlier chunks + these rows)
// is already in the paged cache.  Row j sits at absolute position
// pos = context_lens[s] - L_s + j and attends to cache positions 0..pos.
//
// prefill_generic_kernel: one wave per (row, q-head), any dtype / head_dim /
// block size; each lane owns 4 dims and the keys are visited in order with an
// online softmax.  prefill_mfma_kernel (bf16/f16, head_dim 64/128/256, any GQA ratio) is the
// MFMA tile kernel used whenever it applies; prefill_f32_kernel is its fp32 counterpart on
// v_mfma_f32_32x32x2_f32.
#include <math.h>

#include <algorithm>
#include <type_traits>
#include <utility>

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
  int32_t rank_tiles;  // ceil(max_query_len / 32): tile ranks launched per sequence (MFMA path)
  int32_t sched_kbound;  // > 0: bound on the work keys of the sorted schedule (MFMA path)
  int64_t kv_stride;
  uint32_t kv_stride_bytes;  // MFMA path: block stride in bytes (below 2^32)
  // MFMA path: (kv_stride / (16 D)) << 3 | j for blocks of 16 << j tokens: the block stride in
  // 16-row sub-blocks and the sub-blocks per block (one scalar: the kernel is at its SGPR limit).
  uint32_t win_param;
  // MFMA path, sorted schedule: > 0 when the workgroups of a head group sit three to a CU in
  // sched_cols columns (workgroup q of the group shares its CU with q +- sched_cols): the items
  // are dealt to the columns in snake order and split inside a column by dispatch slot.
  int32_t sched_cols;
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
// Tile = 32 queries of one sequence x one q-head per wave; the 4 waves of a workgroup share the
// K/V tiles of one kv-head: 4 heads on one 32-row tile (GQA 4 and its multiples), 2 heads on
// two consecutive 32-row tiles (GQA 2) or one head on four (no GQA).
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
constexpr int kPWaves = 4;            // waves per workgroup: (heads per workgroup) x (query subtiles)
constexpr int kPThreads = kPWaves * 64;
// Key sub-block of the MFMA path: 16 tokens, two per key tile.  A KV block of 16 << j tokens
// holds 2^j of them (the rows of one kv-head in a block are contiguous, so a sub-block is 16
// consecutive rows of it).
constexpr int kBlk = 16;

typedef short v4i16_t __attribute__((ext_vector_type(4)));

#ifndef RG_PF_STAGES
#define RG_PF_STAGES 3
#endif
// Resident workgroups per CU the persistent grid is sized for (LDS: stages x tile bytes each).
#ifndef RG_PF_WG_PER_CU
#define RG_PF_WG_PER_CU 3
#endif

constexpr int kPStages = RG_PF_STAGES;  // K/V tiles in flight (ring in LDS)
// head_dim 256: the O accumulators (128 VGPRs) and the Q^T operand (64) leave room for one wave
// per SIMD, so one workgroup per CU, with a four-stage ring (4 x 32 KB) to keep three key tiles
// in flight while it computes.
template <int D>
constexpr int pf_wg_per_cu() { return D > 128 ? 1 : RG_PF_WG_PER_CU; }
template <int D>
constexpr int pf_stages() { return D > 128 ? 4 : kPStages; }
// LDS operand reads in flight ahead of the MFMA that uses them: K (QK^T) and V (PV).
#ifndef RG_PF_KAHEAD
#define RG_PF_KAHEAD 4
#endif
#ifndef RG_PF_VAHEAD
#define RG_PF_VAHEAD 3
#endif
constexpr int kKAhead = RG_PF_KAHEAD;
constexpr int kVAhead = RG_PF_VAHEAD;
// Wave priority around the MFMA bursts of the tile loop: 1 while a wave issues its QK or PV
// MFMAs (and the operand reads between them), 0 for its softmax.  Three waves share each SIMD;
// with the priority the one that has MFMAs ready is issued first, so the matrix pipe is fed
// while the others run their softmax in the gaps.
// Column split of the sorted schedule (sched_cols > 0).  The three workgroups of a CU are
// dispatched in order and the oldest wins issue arbitration, so with equal work they end in
// dispatch order, ~27 us apart at config 4 (per-workgroup timestamps): the CU then runs its
// last stretch with one or two workgroups.  Inside a column the items (longest first) go one
// by one to the slot whose finish time (load + item) / rate is least, with the slots' rates
// measured while all three run (0.92 : 0.72 : 0.57 per us at config 4 -> 13 : 10 : 8), an
// item costing its key tiles plus RG_PF_UNIT_COST tiles of unit set-up and epilogue.
#ifndef RG_PF_WEIGHTED
#define RG_PF_WEIGHTED 1
#endif
#ifndef RG_PF_SLOT_W0
#define RG_PF_SLOT_W0 13
#endif
#ifndef RG_PF_SLOT_W1
#define RG_PF_SLOT_W1 10
#endif
#ifndef RG_PF_SLOT_W2
#define RG_PF_SLOT_W2 8
#endif
#ifndef RG_PF_UNIT_COST
#define RG_PF_UNIT_COST 3
#endif
#ifndef RG_PF_PRIO
#define RG_PF_PRIO 1
#endif
// Split softmax: the probabilities of a tile's keys 16..31 are formed while the PV MFMAs of keys
// 0..15 run (interleaved in one wave), instead of all probabilities before the PV product.
#ifndef RG_PF_SPLIT
#define RG_PF_SPLIT 0
#endif
template <int P>
__device__ __forceinline__ void set_wave_prio() {
  if constexpr (RG_PF_PRIO != 0) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(P);
    __builtin_amdgcn_sched_barrier(0);
  }
}
// Sorted schedule tables (LDS): work keys up to kSchedKeys, sequences up to kSchedSeqs.
#ifndef RG_PF_SCHED_KEYS
#define RG_PF_SCHED_KEYS 512
#endif
constexpr int kSchedKeys = RG_PF_SCHED_KEYS;
// Inclusive prefix sum over the 64 lanes with DPP (no LDS round trips): sums within each row
// of 16 lanes by shifts of 1, 2, 4 and 8, then lane 15 of rows 0 and 2 into rows 1 and 3,
// then lane 31 into rows 2 and 3.  Lanes whose source falls outside the row receive 0.
__device__ __forceinline__ int wave_prefix_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}
// Orders this wave's earlier LDS writes before its later LDS reads.
__device__ __forceinline__ void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
constexpr int kSchedSeqs = 256;

constexpr float kSlack = 8.f;           // log2 headroom of the lazy softmax rescale

// acc + lo + hi of a packed pair (v_dot2 with (1, 1), fp32 accumulation).
template <typename T> __device__ __forceinline__ float pair_sum(uint32_t pair, float acc);
template <> __device__ __forceinline__ float pair_sum<bf16_t>(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair),
                                         __builtin_bit_cast(bf16x2_t, 0x3F803F80u), acc, false);
}
template <> __device__ __forceinline__ float pair_sum<f16_t>(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pair), __builtin_bit_cast(f16x2_t, 0x3C003C00u),
                                acc, false);
}

// LDS image of one key tile (two KV blocks of 16 keys).  K: the 16-byte chunk c of key k of
// block b at b * KBYTES / 2 + c * 256 + k * 16, so that one copy instruction (1 KB: chunks
// 4n .. 4n+3 of the block's 16 keys) reads from one block only, and the MFMA A-operand read
// of d chunk i (chunk 2i + half of key j) is one 256-byte run per 16 lanes at a constant
// offset 512 i.  V: row-major [key][D] with the 16-byte chunks of row `key` XOR-swizzled by
// 2*(key & 3) so that the transposing reads of four consecutive rows hit distinct banks.
// (At head_dim 128 the two 16-lane groups that one LDS cycle serves then share 32 banks, a
// 2-way conflict; XOR 4*(key & 3) removes it (bank-conflict cycles / 11) but measured no faster
// at config 4, so the LDS is not what limits the tile loop.)
template <int D>
struct PTile {
  static constexpr int NKC = D / 16;
  static constexpr int KBYTES = NKC * 1024;
  static constexpr int VBYTES = kPT * D * 2;
  static constexpr int BYTES = KBYTES + VBYTES;
  static constexpr int VCHUNKS = D / 8;  // 16-byte chunks per V row
  static constexpr int BLK_INS = D / 32;  // 1 KB copy instructions per block, for K and for V
  __device__ static __forceinline__ int vchunk(int key, int c) { return c ^ (2 * (key & 3)); }
};

template <typename T, int D, int GW>
__global__ __launch_bounds__(kPThreads, pf_wg_per_cu<D>()) void prefill_mfma_kernel(
    PrefillArgs a, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ context_lens, const int32_t* __restrict__ cu_seqlens) {
  using MF = mfma32<T>;
  using S = uint16_t;
  using TL = PTile<D>;
  constexpr int NST = pf_stages<D>();  // ring stages
  // Heads per workgroup GW (1, 2 or 4) and query subtiles QS = 4 / GW: wave w computes head
  // w % GW on query subtile w / GW of the unit, which has UR = 32 * QS rows.
  static_assert(GW == 1 || GW == 2 || GW == 4, "heads per workgroup");
  constexpr int QS = kPWaves / GW;
  constexpr int UR = kPT * QS;
  constexpr int NKC = TL::NKC;     // 16-element d chunks = QK MFMAs per key tile
  constexpr int NDB = D / 32;      // 32-row d blocks of O^T
  // Tile copies: waves 2b and 2b+1 copy block b of the tile, each half of its K and half of
  // its V instructions (BLK_INS / 2 of each).
  constexpr int HALF_INS = TL::BLK_INS / 2;
  static_assert(HALF_INS >= 1 && TL::BLK_INS % 2 == 0, "block copies split over two waves");
  constexpr int LOADS_PER_WAVE = 2 * HALF_INS;
  __shared__ __attribute__((aligned(16))) char lds[NST * TL::BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hkv = a.num_kv_heads;
  const int G = a.num_heads / hkv;
  // Head groups: GW heads of one kv-head each, H / GW of them; group grp is kv-head grp % hkv
  // and its heads hsub * GW .. hsub * GW + GW - 1 within the kv-head (hsub = grp / hkv).
  const int ngroups = a.num_heads / GW;
  // Persistent workgroups: workgroup g serves head group g % ngroups (so, with workgroups
  // placed on the XCDs round-robin, every group of a kv-head lands on the same XCD when
  // hkv is a multiple of 8 and each head's K/V stays in few L2s); the Q = gridDim / ngroups
  // workgroups of a group share its work items, one unit (sequence s, unit tile t of UR rows)
  // each, taken in snake order (round i: position i * Q + q, or i * Q + Q - 1 - q on odd
  // rounds) over a list sorted by work, longest first.  The work key of (s, t) is base_s + t,
  // base_s = ceil(prior_s / UR) + 1 (a unit's key tiles grow by QS per key step), so every key
  // value occurs at most once per sequence: the list is "for k = kmax .. 1, for s ascending
  // with base_s <= k < base_s + nt_s", and position -> (k, s) needs only the count B[k] of
  // items with key >= k (built in LDS once per workgroup) and a scan of the sequences
  // covering k.  Snake order over a work-sorted list keeps the workgroups within a few
  // percent of each other where rank order (all sequences' last tiles first, then the
  // next-to-last ...) left 30 % apart.  Batches beyond the LDS tables (sched_kbound == 0) keep
  // rank order: item (rank r, seq s) = r * num_seqs + s is the r-th unit of s from its end,
  // the last rank taking every unit further from the end (when max_query_len understates a
  // sequence).
  const int grp = blockIdx.x % ngroups;
  const int kvh = grp % hkv;
  const int nq_wg = gridDim.x / ngroups;
  const int qw = blockIdx.x / ngroups;
  const bool sorted = a.sched_kbound > 0;
  const int kb = a.sched_kbound;  // sorted schedule: keys live in [1, kb]
  const int table_tokens = a.max_blocks * a.block_size;
  const int H = a.num_heads;
  const int head = kvh * G + (grp / hkv) * GW + w % GW;
  // This wave's query subtile, w / GW (0 for GW = 4).  Formed where it is used from the thread
  // index behind an empty asm, so that it is not held in a register across the unit loop (the
  // kernel runs at the scalar-register limit).
  auto wave_sub = [&]() -> int {
    if constexpr (QS == 1) {
      return 0;
    } else {
      int t = threadIdx.x;
      asm volatile("" : "+v"(t));
      return __builtin_amdgcn_readfirstlane(t >> 6) / GW;
    }
  };
  const int j = lane & 31;   // query column owned by this lane
  const int hh = lane >> 5;  // which half of the k-slots
  __shared__ int sched_b[kSchedKeys + 2];
  // Sorted schedule, per sequence: its first packed row and the positions cached before its
  // rows (context - rows, negative for an inconsistent context); entry num_seqs holds the end
  // of the packed stream.
  __shared__ int2 sched_seq[kSchedSeqs + 1];
  // Work keys of a sequence of L rows after `prior` cached positions: base ceil(prior / 32) + 1
  // (capped at kb + 1) and the number of its query tiles whose key is within the bound.
  auto seq_keys = [&](int L, int prior) {
    const int nt = L > 0 ? (L + UR - 1) / UR : 0;
    const int bq = min((max(prior, 0) + UR - 1) / UR + 1, kb + 1);
    return make_int2(bq, min(nt, kb + 1 - bq));
  };
  int n_items = a.rank_tiles * a.num_seqs;
  if (sorted) {
    for (int k = tid; k < kb + 2; k += kPThreads) sched_b[k] = 0;
    __syncthreads();
    for (int q = tid; q <= a.num_seqs; q += kPThreads) {
      const int r0 = cu_seqlens[q];
      if (q == a.num_seqs) {
        sched_seq[q] = make_int2(r0, 0);
        continue;
      }
      const int Lq = cu_seqlens[q + 1] - r0;
      const int pr = min(context_lens[q], table_tokens) - Lq;
      sched_seq[q] = make_int2(r0, pr);
      const int2 kn = seq_keys(Lq, pr);  // keys past the bound do not occur (see host)
      if (kn.y > 0) {  // difference array of the per-key counts
        atomicAdd(&sched_b[kn.x], 1);
        atomicAdd(&sched_b[kn.x + kn.y], -1);
      }
    }
    __syncthreads();
    if (w == 0) {
      // counts: prefix sum over k = 1 .. kb; then B[k] = sum of counts over keys >= k.
      int carry = 0;
      for (int c0 = 1; c0 <= kb; c0 += 64) {
        const int k = c0 + lane;
        const int v = wave_prefix_sum(k <= kb ? sched_b[k] : 0) + carry;
        if (k <= kb) sched_b[k] = v;
        carry = __builtin_amdgcn_readlane(v, 63);
      }
      wave_lds_fence();
      carry = 0;
      for (int c1 = kb; c1 >= 1; c1 -= 64) {
        const int k = c1 - lane;
        const int v = wave_prefix_sum(k >= 1 ? sched_b[k] : 0) + carry;
        carry = __builtin_amdgcn_readlane(v, 63);
        if (k >= 1) sched_b[k] = v;
      }
      if (lane == 0) sched_b[kb + 1] = 0;
    }
    __syncthreads();
    n_items = __builtin_amdgcn_readfirstlane(sched_b[1]);
  }
  // This wave's tile copies: block cb of the tile, K instructions n = cp * HALF_INS + t and V
  // instructions cb * BLK_INS + cp * HALF_INS + t (t < HALF_INS).  For each: the key within
  // the tile (copy_key) and the element offset inside its block of the 16 bytes this lane
  // copies (K: key lane & 15, chunk 4n + lane / 16; V: key kl of the instruction, physical
  // chunk swizzled by the row), and the LDS offset of the instruction inside a ring stage.
  const int cb = w >> 1, cp = w & 1;
  auto copy_key_of = [&](int ld, int ln) {
    if (ld < HALF_INS) return kBlk * cb + (ln & (kBlk - 1));
    const int vi = cb * TL::BLK_INS + cp * HALF_INS + ld % HALF_INS;
    return vi * (1024 / (D * 2)) + ln / TL::VCHUNKS;
  };
  auto copy_key = [&](int ld) { return copy_key_of(ld, lane); };
  int32_t lane_off[LOADS_PER_WAVE];
  uint32_t ins_lds[LOADS_PER_WAVE];
#pragma unroll
  for (int ld = 0; ld < LOADS_PER_WAVE; ++ld) {
    const int t = ld % HALF_INS;
    const int kl = copy_key(ld);
    if (ld < HALF_INS) {
      const int n = cp * HALF_INS + t;
      lane_off[ld] = (kl & (kBlk - 1)) * D + 8 * (4 * n + (lane >> 4));
      ins_lds[ld] = cb * (TL::KBYTES / 2) + n * 1024;
    } else {
      const int vi = cb * TL::BLK_INS + cp * HALF_INS + t;
      lane_off[ld] = (kl & (kBlk - 1)) * D + 8 * TL::vchunk(kl, lane % TL::VCHUNKS);
      ins_lds[ld] = TL::KBYTES + vi * 1024;
    }
  }
  // A unit of work: query tile t of sequence s (rows row0 + 32 t ..), whose rows follow
  // `prior` cached positions.  An item of the sorted schedule is one unit; an item of the rank
  // order may hold several (tiles t down to t_stop + 1).
  struct Unit {
    int s, t, t_stop, row0, L, prior;
  };
  // Item u -> its first unit; false for an item without a tile (rank order).
  auto resolve = [&](int u, Unit& un) -> bool {
    if (sorted) {
      // key k: the largest with B[k] > u (B is non-increasing); i: rank of the item among key k's.
      int lo = 1, hi = kb;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sched_b[mid] > u) lo = mid;
        else hi = mid - 1;
      }
      const int k = __builtin_amdgcn_readfirstlane(lo);
      int i = __builtin_amdgcn_readfirstlane(u - sched_b[k + 1]);
      int sq = -1;
      for (int c0 = 0; c0 < a.num_seqs && sq < 0; c0 += 64) {
        const int q = c0 + lane;
        int2 kn = make_int2(0, 0);
        if (q < a.num_seqs) {
          const int2 m0 = sched_seq[q];
          kn = seq_keys(sched_seq[q + 1].x - m0.x, m0.y);
        }
        uint64_t m = __ballot(kn.x <= k && k < kn.x + kn.y);
        const int cnt = __builtin_popcountll(m);
        if (i < cnt) {
          for (; i > 0; --i) m &= m - 1;
          sq = c0 + __ffsll((unsigned long long)m) - 1;
        } else {
          i -= cnt;
        }
      }
      un.s = __builtin_amdgcn_readfirstlane(sq);
      if (un.s < 0) return false;  // (not reached with consistent tables)
      const int2 m0 = sched_seq[un.s];
      un.row0 = __builtin_amdgcn_readfirstlane(m0.x);
      un.L = __builtin_amdgcn_readfirstlane(sched_seq[un.s + 1].x) - un.row0;
      un.prior = __builtin_amdgcn_readfirstlane(m0.y);
      un.t = k - seq_keys(un.L, un.prior).x;
      un.t_stop = un.t - 1;
      return true;
    }
    un.s = u % a.num_seqs;
    const int rank = u / a.num_seqs;
    un.row0 = cu_seqlens[un.s];
    un.L = cu_seqlens[un.s + 1] - un.row0;
    const int nts = (un.L + UR - 1) / UR;
    if (rank >= nts) return false;
    un.prior = min(context_lens[un.s], table_tokens) - un.L;
    un.t = nts - 1 - rank;
    un.t_stop = rank == a.rank_tiles - 1 ? -1 : un.t - 1;
    return true;
  };
  // Work items of this workgroup, in snake order (round r: position r * Q + q, or
  // r * Q + Q - 1 - q on odd rounds, for the Q workgroups of the kv-head); n_items once done.
  // (A shared work counter was measured: it evens out the workgroups of a CU but not the
  // CU's finish time, and its round trips cost more than it saved.)
  // With columns (sched_cols = C > 0) the snake runs over the C columns instead (round r of
  // column c: position r * C + c, or r * C + C - 1 - c), and the column's first 64 rounds are
  // split between its three workgroups (slot qw / C, dispatch order) by the weighted greedy
  // of RG_PF_SLOT_W*, which every workgroup of the column computes alike from its own copy of
  // the tables.  Rounds from 64 on go to the slots in turn.  Each wave keeps this state in LDS,
  // not in registers (the kernel is at its scalar-register limit): the rounds of the first 64
  // it has not yet taken (`sched_mine`) and (C, column, its next round from 64 on).  Rounds 0, 1
  // and 2 go to slots 0, 1 and 2 (what the greedy gives anyway for items longest first when
  // F0 < F1 < F2 < 2 F0), so a workgroup knows its first item before the greedy runs: it
  // resolves that item and sends its loads out first, and the greedy runs while they are in
  // flight.
  __shared__ uint64_t sched_mine[kPWaves];
  __shared__ int4 sched_colw[kPWaves];
  const int cols = sorted ? a.sched_cols : 0;
  if (cols == 0) sched_colw[w] = make_int4(0, 0, 0, 0);
  int round = 0;
  auto take_item = [&]() -> int {
    const int4 cw = sched_colw[w];
    if (cw.x > 0) {
      int r;
      const uint64_t mine = sched_mine[w];
      if (mine != 0) {
        r = __builtin_ctzll(mine);
        sched_mine[w] = mine & (mine - 1);
      } else {
        r = cw.z;
        sched_colw[w].z = r + 3;
      }
      const int u = r * cw.x + ((r & 1) ? cw.x - 1 - cw.y : cw.y);
      return u < n_items ? u : n_items;
    }
    const int r = round++;
    const int u = r * nq_wg + ((r & 1) ? nq_wg - 1 - qw : qw);
    return u < n_items ? u : n_items;
  };

  // Per-unit registers, loaded ahead of the unit: the block-table window and the Q^T operand
  // (lane holds q[query j][16i + 8hh .. +8] for every d chunk i; a row without a position
  // holds the unit's first row instead: its scores stay finite and its output is written as
  // zeros, and no select on the loaded value makes the load wait where it is issued).  Window: lane i holds the cache addresses, in units of 16 rows (16 D elements),
  // of this kv-head's rows of 16-token sub-blocks 2 wb + i and 2 wb + 64 + i (clamped to the
  // unit's last sub-block), i.e. of key tiles wb .. wb + 63, so a tile's two sub-block addresses
  // are v_readlane's and a copy's address is one multiply by a constant.  Sub-block v lies in
  // block table entry v >> bs_shift, at row 16 (v & (2^bs_shift - 1)) of the kv-head's rows.
  int btw0 = 0, btw1 = 0;
  uint4 qb[NKC];
  auto load_window = [&](const Unit& un, int wbase, int last_sub) {
    const int32_t* bt = block_table + (int64_t)un.s * a.max_blocks;
    // (Derived here from the one packed argument behind an empty asm, not hoisted into scalar
    // registers that would stay live across the unit loop.)
    uint32_t wp = a.win_param;
    asm volatile("" : "+s"(wp));
    const int sh = (int)(wp & 7u);
    const int v0 = min(2 * wbase + lane, last_sub), v1 = min(2 * wbase + 64 + lane, last_sub);
    // The raw block numbers: finish_window turns them into addresses once they have landed, so
    // no wait for them falls where the loads are issued (the set-up, or before an epilogue).
    btw0 = bt[v0 >> sh];
    btw1 = bt[v1 >> sh];
  };
  // Unsigned 32-bit: the address of the pool's last row in units of 16 D elements is below
  // 2^32 for any pool the device holds (2^32 * 32 D bytes is 8 TB at head_dim 64).
  auto finish_window = [&](int wbase, int last_sub) {
    uint32_t wp = a.win_param;
    asm volatile("" : "+s"(wp));
    const int sh = (int)(wp & 7u);
    const int v0 = min(2 * wbase + lane, last_sub), v1 = min(2 * wbase + 64 + lane, last_sub);
    const uint32_t head = (uint32_t)kvh << sh;  // the kv-head's first sub-block within a block
    const uint32_t spb = wp >> 3, sm = (1u << sh) - 1u;
    btw0 = (int)((uint32_t)btw0 * spb + head + ((uint32_t)v0 & sm));
    btw1 = (int)((uint32_t)btw1 * spb + head + ((uint32_t)v1 & sm));
  };
  auto load_unit = [&](const Unit& un) {
    const int q0 = un.t * UR;
    const int pos_max = un.prior + q0 + min(UR, un.L - q0) - 1;
    const int wq0 = q0 + kPT * wave_sub();  // this wave's first row
    const bool row_ok = j < un.L - wq0 && un.prior + wq0 + j >= 0;
    if (pos_max >= 0) load_window(un, 0, pos_max / kBlk);
    const uint4* qr = reinterpret_cast<const uint4*>(q + ((int64_t)(un.row0 + (row_ok ? wq0 + j : 0)) * H + head) * D);
#pragma unroll
    for (int i = 0; i < NKC; ++i) qb[i] = qr[2 * i + hh];
  };

  Unit cur{};
  bool have = false;
  if (cols > 0) {
    const int col = qw % cols, slot = qw / cols;
    const int u = slot * cols + ((slot & 1) ? cols - 1 - col : col);  // round `slot` of the column
    have = u < n_items && resolve(u, cur);
  } else {
    for (int u = take_item(); u < n_items; u = take_item()) {
      if (resolve(u, cur)) {
        have = true;
        break;
      }
    }
  }
  if (have) load_unit(cur);
  // The split is computed by wave 0 alone, for the four waves (the greedy is a chain of scalar
  // instructions, and the CU's scalar unit serves all its waves), then published with a barrier
  // that waits for the LDS writes only (__syncthreads would also wait for the first unit's
  // loads, which are to land during the greedy).
  if (cols > 0 && w == 0) {
    const int col = qw % cols, slot = qw / cols;
    uint64_t mine = 0;
    const int u = lane * cols + ((lane & 1) ? cols - 1 - col : col);
    int cost = 0;
    if (u < n_items) {
      int lo = 1, hi = kb;  // the item's key, as in resolve
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sched_b[mid] > u) lo = mid;
        else hi = mid - 1;
      }
      cost = lo * QS + RG_PF_UNIT_COST;
    }
    constexpr int F0 = RG_PF_SLOT_W1 * RG_PF_SLOT_W2, F1 = RG_PF_SLOT_W0 * RG_PF_SLOT_W2,
                  F2 = RG_PF_SLOT_W0 * RG_PF_SLOT_W1;
    int l0 = 0, l1 = 0, l2 = 0;
    for (int i = 0; i < 64; ++i) {
      const int c = __builtin_amdgcn_readlane(cost, i);
      if (c == 0) break;  // past the column's last item
      // Finish times (l_s + c) / w_s, compared as (l_s + c) * (product of the other weights),
      // times 4 plus the slot: one minimum picks the slot, ties going to the lower one, all in
      // scalar instructions.  (< 2^31: l_s + c <= 64 (4 kb + 3).)
      const int sl = i < 3 ? i
                           : min(min((l0 + c) * (4 * F0), (l1 + c) * (4 * F1) + 1), (l2 + c) * (4 * F2) + 2) & 3;
      l0 += sl == 0 ? c : 0;
      l1 += sl == 1 ? c : 0;
      l2 += sl == 2 ? c : 0;
      mine |= (uint64_t)(sl == slot) << i;
    }
    if (lane < kPWaves) {
      sched_mine[lane] = mine & ~(1ull << slot);  // round `slot`: the first item, already taken
      sched_colw[lane] = make_int4(cols, col, 64 + slot, 0);
    }
  }
  if (cols > 0) {
    wave_lds_fence();
    tile_barrier();
  }

  while (have) {
  const int row0 = cur.row0;
  const int q0 = cur.t * UR;                   // first query of the unit (within the sequence)
  const int pos_max = cur.prior + q0 + min(UR, cur.L - q0) - 1;  // the unit's last position
  const int wq0 = q0 + kPT * wave_sub();       // this wave's first query
  const int nq = min(kPT, cur.L - wq0);        // this wave's rows (<= 0: none)
  const int pos_min = cur.prior + wq0;
  const bool row_ok = j < nq && pos_min + j >= 0;
  // Rows without a position attend like the tile's last row (finite scores; written as zeros).
  const int my_pos = row_ok ? pos_min + j : pos_max;
  int wb = 0;
  // Q and the window have landed; nothing else is in flight.
  __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);  // vmcnt(0)
  if (pos_max >= 0) finish_window(0, pos_max / kBlk);
  constexpr uint32_t kSubBytes = kBlk * D * 2;  // one window unit: 16 rows
  const int nkt = pos_max >= 0 ? pos_max / kPT + 1 : 0;
  const uint32_t lds_base = (uint32_t)(uintptr_t)((RG_LDS char*)lds);

  // Issues this wave's share of the global->LDS copies of key tile kt (wb <= kt < wb + 64)
  // into ring stage st.  Keys past the last position read the last valid key instead (they
  // are masked).  Every instruction reads from one block (this wave's block cb of the tile),
  // so the fast path is a scalar block base (block number x block stride, 32 x 32 -> 64-bit)
  // plus the lane's fixed 32-bit offset; only the last tile of an item needs the clamp to
  // pos_max, with per-lane addresses (the slow path).
  auto issue_tile = [&](int kt, int st) {
    const int r = 2 * (kt - wb);  // even: both blocks sit in the same window register
    // (The stage base is formed here from an opaque copy of the LDS base: hoisted, every
    // (stage, copy) pair of the unrolled ring kept its own M0 value in a scalar register, 32 at
    // head_dim 256.)
    uint32_t lb = lds_base;
    asm volatile("" : "+s"(lb));
    const uint32_t sbase = lb + st * TL::BYTES;
    if (kt * kPT + kPT - 1 <= pos_max) {
      const uint32_t e = (uint32_t)__builtin_amdgcn_readlane(r < 64 ? btw0 : btw1, (r & 63) + cb);
      const uint64_t boff = (uint64_t)e * kSubBytes;
      const char* kbase = reinterpret_cast<const char*>(kc) + boff;
      const char* vbase = reinterpret_cast<const char*>(vc) + boff;
#pragma unroll
      for (int ld = 0; ld < LOADS_PER_WAVE; ++ld) {
        lds_dma16_s(ld < HALF_INS ? kbase : vbase, (uint32_t)lane_off[ld] * 2u, sbase + ins_lds[ld]);
      }
      return;
    }
    const int e0 = __builtin_amdgcn_readlane(r < 64 ? btw0 : btw1, r & 63);
    const int e1 = __builtin_amdgcn_readlane(r < 64 ? btw0 : btw1, (r & 63) + 1);
    const int64_t blk0 = (int64_t)(uint32_t)e0 * (kBlk * D);
    const int64_t blk1 = (int64_t)(uint32_t)e1 * (kBlk * D);
    // (The lane's keys are formed here from an opaque copy of the lane index, not kept from the
    // set-up: this path runs once per unit and the registers are all taken around it.)
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int ld = 0; ld < LOADS_PER_WAVE; ++ld) {
      // The copy of key lane_key (within the tile) with the clamped key's row instead.
      const int kl = copy_key_of(ld, ln);
      const int key = min(kt * kPT + kl, pos_max) - kt * kPT;
      const int64_t src = (key < kBlk ? blk0 : blk1) + (int64_t)((key & (kBlk - 1)) - (kl & (kBlk - 1))) * D +
                          lane_off[ld];
      lds_dma16((ld < HALF_INS ? kc : vc) + src, sbase + ins_lds[ld]);
    }
  };

  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  // m_run + kSlack in raw score units (this path runs with scale > 0 only), so that a tile's
  // test needs no multiply: raw maximum > m_thr  <=>  scaled maximum > m_run + kSlack.
  float m_thr = -INFINITY;

  // The tile loop runs each tile in order (scores, maximum, probabilities, PV); the overlap
  // of one wave's softmax with another's MFMAs comes from the three workgroups sharing each
  // SIMD.  Ring: iteration kt reads tile kt's K and V from its stage; copies of tiles
  // kt+1 .. kt+NST-1 are in flight (tile kt+NST-1 issued during kt's QK MFMAs into
  // the stage tile kt-1 left).
  static_assert(NST >= 3 && NST <= 64, "ring depth");
  const char* vlds = lds + TL::KBYTES;
  const int grp = lane >> 4;
  const int e_row = (lane >> 2) & 3;
  const int qq = lane & 3;
  // Tiles from here on may hold keys past one of this wave's queries (a wave without rows
  // masks against the unit's last position).
  const int kt_mask = (QS == 1 ? pos_min : min(pos_min, pos_max)) / kPT;
  // With several row subtiles per unit (QS > 1) the unit's tiles run to its last row, past this
  // wave's own last row: from tile kt_last + 1 on every key lies beyond all of this wave's rows,
  // so the tile would add exact zeros (p = 0) and the wave only takes part in its copies and
  // barrier, leaving the SIMD to the CU's other workgroups.  (-1: no row with a position.)
  const int wave_last = pos_min + nq - 1;
  const int kt_last = QS > 1 && nq > 0 && wave_last >= 0 ? wave_last / kPT : QS > 1 ? -1 : nkt;
  const int xor32_addr = (lane ^ 32) << 2;  // ds_bpermute address of the other half's lane

  // S^T = K Q^T of the tile in stage st: c[4jb + r] is key 8jb + 4hh + r for query j.  The K
  // operands are read kKAhead MFMAs ahead of their use (a rolling set of registers); the
  // scheduling barriers keep that order, which the compiler would otherwise trade for fewer
  // registers by waiting for each read right before its MFMA.
  const int k_lane = (j >> 4) * (TL::KBYTES / 2) + hh * 256 + (j & (kBlk - 1)) * 16;
  auto scores = [&](int st) {
    const char* base = lds + st * TL::BYTES + k_lane;
    constexpr int A = kKAhead < NKC ? kKAhead : NKC;
    uint4 ka[A];
#pragma unroll
    for (int i = 0; i < A; ++i) ka[i] = *reinterpret_cast<const uint4*>(base + i * 512);
    f32x16_t c;
#pragma unroll
    for (int v = 0; v < 16; ++v) c[v] = 0.f;
#pragma unroll
    for (int i = 0; i < NKC; ++i) {
      __builtin_amdgcn_sched_barrier(0);
      c = MF::run(ka[i % A], qb[i], c);
      if (i + A < NKC) ka[i % A] = *reinterpret_cast<const uint4*>(base + (i + A) * 512);
    }
    __builtin_amdgcn_sched_barrier(0);
    return c;
  };
  // Masks keys past each query's position (tiles from kt_mask on, branch-free) and returns
  // the raw maximum of this lane's half of the query's keys.
  auto mask_max = [&](f32x16_t& c, int kt) {
    if (kt >= kt_mask) {  // wave-uniform: only the tiles around the diagonal hold such keys
      // key 8 (v >> 2) + 4 hh + (v & 3) > my_pos - 32 kt, with the lane's part on the right
      // so that the left side is an inline constant.
      const int lim = my_pos - kt * kPT - 4 * hh;
#pragma unroll
      for (int v = 0; v < 16; ++v) c[v] = 8 * (v >> 2) + (v & 3) > lim ? -INFINITY : c[v];
    }
    float tmax = c[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) tmax = fmaxf(tmax, c[v]);
    return tmax;
  };
  // Online softmax with a lazy maximum: m_run only moves when a tile's maximum exceeds it by
  // more than kSlack, so p = 2^(x - m_run) stays below 2^kSlack and the O^T rescale is rare.
  // Each lane checks its own half of the query's keys; only when some lane's half exceeds the
  // slack do the two halves (lanes l and l ^ 32, which must keep the same m_run because the
  // PV product sums over both) exchange their maxima.
  auto update_max = [&](float raw_half) {
    if (__ballot(raw_half > m_thr)) {
      const float other = __int_as_float(__builtin_amdgcn_ds_bpermute(xor32_addr, __float_as_int(raw_half)));
      const float tmax = fmaxf(raw_half, other) * a.scale_log2;
      const bool grow = tmax > m_run + kSlack;
      const float m_new = grow ? tmax : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      m_thr = (m_run + kSlack) / a.scale_log2;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
    }
  };
  // Probabilities of tile scores c as the packed B operand of the PV product (keys 16n+4hh+r
  // and 16n+8+4hh+r in k-slots 8hh..8hh+7 for n = 0, 1).
  // The row sum adds the rounded pairs (two dot products with (1, 1)), so the normaliser
  // weighs exactly the probabilities that enter the PV product.
  auto probs = [&](const f32x16_t& c, uint32_t (&pk)[8]) {
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(c[v], a.scale_log2, -m_run));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(c[v + 1], a.scale_log2, -m_run));
      pk[v / 2] = pack2<T>(p0, p1);
    }
    // Two chains, the first one starting from l_run itself.
    float s0 = pair_sum<T>(pk[0], l_run), s1 = pair_sum<T>(pk[1], 0.f);
#pragma unroll
    for (int i = 2; i < 8; i += 2) {
      s0 = pair_sum<T>(pk[i], s0);
      s1 = pair_sum<T>(pk[i + 1], s1);
    }
    l_run = s0 + s1;
  };
  // The probabilities of keys 16h .. 16h + 15 only (scores c[8h .. 8h + 7]) into pk[4h .. 4h + 3],
  // their row sum added to l_run.
  auto probs_half = [&](const f32x16_t& c, int h, uint32_t (&pk)[8]) {
#pragma unroll
    for (int v = 8 * h; v < 8 * h + 8; v += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(c[v], a.scale_log2, -m_run));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(c[v + 1], a.scale_log2, -m_run));
      pk[v / 2] = pack2<T>(p0, p1);
    }
    const float s0 = pair_sum<T>(pk[4 * h + 2], pair_sum<T>(pk[4 * h], l_run));
    const float s1 = pair_sum<T>(pk[4 * h + 3], pair_sum<T>(pk[4 * h + 1], 0.f));
    l_run = s0 + s1;
  };
  // O^T += V^T P^T for the tile in stage st, in two 16-key MFMA steps.  The A operand comes
  // from the transposing LDS read: in each 16-lane group, lane 4e+q points at
  // V[key0 + e][d0 + 4q .. +4] and lane i receives V[key0 .. key0+3][d0 + i].
  // A operand m = n * NDB + db of the PV product (keys 16n .. 16n+15, d block db).
  auto v_operand = [&](int st, int m) {
    const char* vbase = vlds + st * TL::BYTES;
    const int n = m / NDB, db = m % NDB;
    const int d = 32 * db + 16 * (grp & 1) + 4 * qq;  // this lane's address column
    v4i16_t part[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int key = 16 * n + 8 * half + 4 * (grp >> 1) + e_row;
      const int off = key * (D * 2) + TL::vchunk(key, d >> 3) * 16 + (d & 7) * 2;
      part[half] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((RG_LDS v4i16_t*)(vbase + off));
    }
    const uint2 lo = __builtin_bit_cast(uint2, part[0]);
    const uint2 hi = __builtin_bit_cast(uint2, part[1]);
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
  };
  // The first kVAhead V operands are read before the softmax (their latency hides under it),
  // the rest kVAhead MFMAs ahead of use, in a rolling set of registers.
  constexpr int kVA = kVAhead < 2 * NDB ? kVAhead : 2 * NDB;
  auto v_prefetch = [&](int st, uint4 (&va)[kVA]) {
#pragma unroll
    for (int m = 0; m < kVA; ++m) va[m] = v_operand(st, m);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto accumulate = [&](int st, const uint32_t (&pk)[8], uint4 (&va)[kVA]) {
#pragma unroll
    for (int m = 0; m < 2 * NDB; ++m) {
      const int n = m / NDB;
      const uint4 pb = make_uint4(pk[4 * n], pk[4 * n + 1], pk[4 * n + 2], pk[4 * n + 3]);
      __builtin_amdgcn_sched_barrier(0);
      o[m % NDB] = MF::run(va[m % kVA], pb, o[m % NDB]);
      if (m + kVA < 2 * NDB) va[m % kVA] = v_operand(st, m + kVA);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // accumulate with the probabilities of keys 16..31 formed under the PV MFMAs of keys 0..15
  // (pk[0..3] are ready on entry).
  auto accumulate_split = [&](int st, const f32x16_t& c, uint32_t (&pk)[8], uint4 (&va)[kVA]) {
    const uint4 pb0 = make_uint4(pk[0], pk[1], pk[2], pk[3]);
#pragma unroll
    for (int m = 0; m < NDB; ++m) {
      o[m] = MF::run(va[m % kVA], pb0, o[m]);
      if (m + kVA < 2 * NDB) va[m % kVA] = v_operand(st, m + kVA);
    }
    probs_half(c, 1, pk);
#pragma unroll
    for (int m = 0; m < NDB; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // six VALU
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two LDS reads
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint4 pb1 = make_uint4(pk[4], pk[5], pk[6], pk[7]);
#pragma unroll
    for (int m = NDB; m < 2 * NDB; ++m) {
      __builtin_amdgcn_sched_barrier(0);
      o[m % NDB] = MF::run(va[m % kVA], pb1, o[m % NDB]);
      if (m + kVA < 2 * NDB) va[m % kVA] = v_operand(st, m + kVA);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // This wave's copies of tile `need` have landed (all but the newest `pending` groups),
  // then the barrier shows every wave's copies and retires the stages read before it.
  auto wait_tiles = [&](auto pending) {
    constexpr int n = LOADS_PER_WAVE * decltype(pending)::value;
    static_assert(n < 64, "vmcnt immediate (6 bits: [3:0] and [15:14])");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | 0x70 | 0xF00);
    tile_barrier();
  };

  // In-order tile loop: the copies of tiles kt .. min(kt + NST - 2, nkt - 1) are in flight
  // when iteration kt starts; once tile kt has landed everywhere (wait + barrier, which also
  // shows every wave is done with tile kt - 1), stage (kt - 1) % NST takes tile
  // kt + NST - 1 (if there is one), then tile kt is computed: scores, maximum,
  // probabilities, PV.
  static_assert(NST == 3 || NST == 4, "ring depth");
  auto wait_for = [&](int kt) {  // tile kt landed; min(NST - 2, nkt - 1 - kt) newer tiles may not have
    const int newer = nkt - 1 - kt;
    if (newer >= NST - 2) wait_tiles(std::integral_constant<int, NST - 2>{});
    else if (NST == 4 && newer == 1) wait_tiles(std::integral_constant<int, 1>{});
    else wait_tiles(std::integral_constant<int, 0>{});
  };
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    if (p < nkt) issue_tile(p, p);
  // Next unit (the next tile of this item, or the first unit of the next item), found while
  // the first copies are in flight: it needs only the LDS tables and the static item order.
  Unit nxt{};
  bool nhave = false;
  if (cur.t - 1 > cur.t_stop) {
    nxt = cur;
    nxt.t = cur.t - 1;
    nhave = true;
  } else {
    for (int u = take_item(); u < n_items; u = take_item()) {
      if (resolve(u, nxt)) {
        nhave = true;
        break;
      }
    }
  }
  // Tile kt in ring stage SC (a compile-time stage).
  auto tile_step = [&](int kt, auto sc) __attribute__((always_inline)) {
    constexpr int S = decltype(sc)::value;
    wait_for(kt);
    set_wave_prio<1>();
    f32x16_t c = scores(S);
    // The copies of tile kt + NST - 1 go out while the QK MFMAs run.
    if (kt + NST - 1 < nkt) issue_tile(kt + NST - 1, S == 0 ? NST - 1 : S - 1);
    uint4 va[kVA];
    v_prefetch(S, va);
    set_wave_prio<0>();
    update_max(mask_max(c, kt));
    uint32_t pk[8];
    if constexpr (RG_PF_SPLIT != 0) {
      probs_half(c, 0, pk);
      set_wave_prio<1>();
      accumulate_split(S, c, pk, va);
    } else {
      probs(c, pk);
      set_wave_prio<1>();
      accumulate(S, pk, va);
    }
    set_wave_prio<0>();
  };
  int kt = 0;
  int st = 0;  // ring stage of tile kt (kt % NST, kept as a rotating counter)
  while (kt < nkt) {
  // Iterations whose refill tile kt + NST - 1 lies in the current block-table window.
  const int kend = min(nkt, wb + 65 - NST);
  for (; kt < min(kend, kt_last + 1); ++kt) {
    // One copy of the tile per ring stage, so that each stage's LDS offsets are immediates.
    [&]<int... S>(std::integer_sequence<int, S...>) {
      ((st == S ? tile_step(kt, std::integral_constant<int, S>{}) : void()), ...);
    }(std::make_integer_sequence<int, NST>{});
    st = st == NST - 1 ? 0 : st + 1;
  }
  if constexpr (QS > 1) {
    for (; kt < kend; ++kt) {  // tiles past this wave's rows: its copies and the barrier only
      wait_for(kt);
      if (kt + NST - 1 < nkt) issue_tile(kt + NST - 1, st == 0 ? NST - 1 : st - 1);
      st = st == NST - 1 ? 0 : st + 1;
    }
  }
  if (kt >= nkt) break;
  wb += 64;
  load_window(cur, wb, pos_max / kBlk);
  __builtin_amdgcn_s_waitcnt(0x70 | 0xF00);  // vmcnt(0)
  finish_window(wb, pos_max / kBlk);
  }

  // Every wave is done with the LDS stages after the barrier; the next unit's Q and window
  // loads go out before this unit's epilogue.
  tile_barrier();
  // Normalise (the two halves of a query's keys live in lanes l and l ^ 32) and write; rows
  // without a position get zeros.  The tile goes out through LDS, DP columns at a time: each
  // wave writes its rows into its quarter of ring stage NST - 1 (16-byte chunks XOR-
  // swizzled by the row), then reads whole row pieces back, so that every store writes
  // 16 bytes per lane over full runs of a row.  That stage is free here: after the barrier
  // above nobody reads the ring, the next unit's prologue fills stages 0 and 1, and stage
  // NST - 1 is refilled only after the next unit's first barrier.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = row_ok ? 1.f / l_tot : 0.f;
  if (nhave) load_unit(nxt);
  {
    constexpr int DP = TL::BYTES / kPWaves / (kPT * 2);  // columns per pass
    constexpr int CH = DP / 8;                            // 16-byte chunks per row piece
    constexpr int RPR = 64 / CH;                          // rows per read
    static_assert(D % DP == 0 && DP % 32 == 0 && 64 % CH == 0, "epilogue passes");
    char* ebuf = lds + (NST - 1) * TL::BYTES + w * (TL::BYTES / kPWaves);
    // (The lane's rows are formed here, not hoisted out of the unit loop, where they would
    // take registers for the whole loop.)
    int lr = lane;
    asm volatile("" : "+v"(lr));
    const int wr = lr & 31;  // row written by this lane (its query column j)
#pragma unroll
    for (int pass = 0; pass < D / DP; ++pass) {
#pragma unroll
      for (int db = pass * DP / 32; db < (pass + 1) * DP / 32; ++db)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const int dl = 32 * db + 8 * jb - pass * DP;  // + 4 hh
          const uint32_t w0 = pack2<T>(o[db][4 * jb] * inv, o[db][4 * jb + 1] * inv);
          const uint32_t w1 = pack2<T>(o[db][4 * jb + 2] * inv, o[db][4 * jb + 3] * inv);
          const int off = wr * (DP * 2) + (((dl >> 3) ^ (wr & (CH - 1))) << 4) + 8 * (lr >> 5);
          *reinterpret_cast<uint2*>(ebuf + off) = make_uint2(w0, w1);
        }
      wave_lds_fence();
#pragma unroll
      for (int i = 0; i < kPT / RPR; ++i) {
        const int r = i * RPR + lr / CH, c = lr % CH;
        const uint4 v = *reinterpret_cast<const uint4*>(ebuf + r * (DP * 2) + ((c ^ (r & (CH - 1))) << 4));
        if (r < nq) {
          S* orow = static_cast<S*>(a.out) + ((int64_t)(row0 + wq0 + r) * H + head) * D;
          *reinterpret_cast<uint4*>(orow + pass * DP + 8 * c) = v;
        }
      }
      wave_lds_fence();  // the reads have returned before the next pass overwrites the buffer
    }
  }
  cur = nxt;
  have = nhave;
  }  // units of this workgroup
}

// ------------------------------------------------------------ fp32 MFMA tile kernel --
//
// The reference's element type.  fp32 MFMA (v_mfma_f32_32x32x2_f32) is 16x slower per flop
// than bf16 and the kernel is bound by it.  Units are tiles of UR query rows of one sequence
// for GW heads of one kv-head (as in prefill_mfma_kernel: GW = min(G, 4) heads, 4 / GW
// subtiles of 32 rows); workgroup (r, s, group) of the grid takes the units r, r + R, ... of
// sequence s (R = gridDim.x).  The 32-key K and V tiles reach LDS by direct global -> LDS
// copies into two buffers, tile kt + 1 in flight while tile kt computes.
//
//  * Scores transposed, S^T = K Q^T: lane (row l % 32, half h = l / 32) provides K[key l % 32]
//    and Q[query l % 32] at the d of MFMA k-index h; inside a pair of steps the d order is
//    permuted (k-index 0 <-> d = 4c + e, 1 <-> 4c + 2 + e), the same for both operands, so a
//    lane reads its two K values of steps (c, 0) and (c, 1) as one 8-byte LDS read (K tile
//    stored as [d / 4][key][4 floats]).  Q (scaled by scale * log2 e) stays in registers.
//  * The output S^T[key][query] leaves lane l the query l % 32 and keys 8 j + 4 h + r, so the
//    softmax statistics are per lane (the two halves of a query's 32 keys meet through one
//    lane exchange).
//  * O^T = V^T P^T: step (j, r) pairs keys 8 j + r (k-index 0) and 8 j + 4 + r (k-index 1),
//    which are exactly the P values lane halves 0 and 1 hold in register (j, r); the V^T
//    operand is 32 consecutive floats of a V row per half-wave (V tile row-major in LDS).
//    Lane l accumulates O[query l % 32][d block b: 8 j + 4 h + r].
template <int D, int GW>
__global__ __launch_bounds__(kPThreads, D > 128 ? 1 : 2) void prefill_f32_kernel(PrefillArgs a) {
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  constexpr int QS = kPWaves / GW;      // 32-row subtiles per unit
  constexpr int UR = kPT * QS;          // rows per unit
  constexpr int NC = D / 4;             // 16-byte pieces per row
  constexpr int NDB = D / 32;           // d blocks of the output
  constexpr int TILE = kPT * D;         // floats per K (or V) tile
  constexpr int PER = TILE / 4 / kPThreads;  // copies per wave per operand and tile
  static_assert(PER * 4 * kPThreads == TILE, "tile pieces per thread");
  __shared__ __attribute__((aligned(16))) float k_lds[2][TILE];
  __shared__ __attribute__((aligned(16))) float v_lds[2][TILE];
  const uint32_t k_base = (uint32_t)(uintptr_t)((RG_LDS float*)&k_lds[0][0]);
  const uint32_t v_base = (uint32_t)(uintptr_t)((RG_LDS float*)&v_lds[0][0]);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qi = lane & 31, h = lane >> 5;
  const int s = blockIdx.y;
  const int G = a.num_heads / a.num_kv_heads;
  const int head = blockIdx.z * GW + (w % GW);
  const int kvh = (blockIdx.z * GW) / G;
  const int sub = w / GW;
  const int row0 = a.cu_seqlens[s];
  const int L = a.cu_seqlens[s + 1] - row0;
  const int ctx = a.context_lens[s];
  const int first = ctx - L;           // position of the sequence's first new row
  const float* q = static_cast<const float*>(a.q);
  const float* kc = static_cast<const float*>(a.k_cache);
  const float* vc = static_cast<const float*>(a.v_cache);
  float* out = static_cast<float*>(a.out);
  const int32_t* bt = a.block_table + (int64_t)s * a.max_blocks;
  int bs = a.block_size;
  int key_cap = a.max_blocks * bs;  // positions the table row can address
  int first_v = first;
  // Per-lane arithmetic only: kept in VGPRs (the scalar registers are the tight budget here).
  asm volatile("" : "+v"(bs), "+v"(key_cap), "+v"(first_v));

  for (int unit = blockIdx.x; unit * UR < L; unit += gridDim.x) {
    const int myrow = unit * UR + sub * kPT + qi;
    const bool row_ok = myrow < L;
    const int qpos = first_v + myrow;           // negative: a row without a position (zeros)
    // Keys of the unit: positions 0 .. (position of its last row), within the context.
    const int last_row = min(unit * UR + UR, L) - 1;
    const int nkeys = __builtin_amdgcn_readfirstlane(max(0, min(min(ctx, key_cap), first_v + last_row + 1)));
    const int ntiles = (nkeys + kPT - 1) / kPT;

    // Copies of tile kt into buffer kt % 2: copy i of wave w moves LDS pieces
    // 64 (w PER + i) + lane; keys past the unit's last read the last one (masked below).  The
    // block-table reads come first, so that no wait for one of them falls between copies.
    auto issue = [&](int kt) __attribute__((always_inline)) {
      const uint32_t off = (uint32_t)((kt & 1) * TILE * 4);
      int64_t ksrc[PER], vsrc[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int pc = 64 * (w * PER + i) + lane;
        const int kk = min(kt * kPT + pc % kPT, nkeys - 1);   // K image [d / 4][key][4]
        ksrc[i] = (int64_t)bt[kk / bs] * a.kv_stride + ((int64_t)kvh * bs + kk % bs) * D + 4 * (pc / kPT);
        const int vk = min(kt * kPT + pc / NC, nkeys - 1);     // V image row-major
        vsrc[i] = (int64_t)bt[vk / bs] * a.kv_stride + ((int64_t)kvh * bs + vk % bs) * D + 4 * (pc % NC);
      }
      // Every address is formed (the compiler's waits for the table reads placed) before the
      // first copy: a wait it placed after a copy would wait for that copy too.
#pragma unroll
      for (int i = 0; i < PER; ++i) asm volatile("" ::"v"(ksrc[i]), "v"(vsrc[i]));
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const uint32_t dst = off + (uint32_t)(64 * (w * PER + i)) * 16;
        lds_dma16(kc + ksrc[i], k_base + dst);
        lds_dma16(vc + vsrc[i], v_base + dst);
      }
    };

    float qr[NC][2];
    {
      const int row = min(myrow, L - 1);
      const float* qp = q + ((int64_t)(row0 + row) * a.num_heads + head) * D;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float2 v = *reinterpret_cast<const float2*>(qp + 4 * c + 2 * h);
        qr[c][0] = v.x * a.scale_log2;
        qr[c][1] = v.y * a.scale_log2;
      }
    }
    f32x16 o[NDB];
#pragma unroll
    for (int b = 0; b < NDB; ++b) o[b] = f32x16{};
    float m = -INFINITY, lsum = 0.f;

    // With several row subtiles per unit (QS > 1) every key of tiles past kfull lies beyond this
    // wave's own rows (their probabilities are exact zeros): there the wave only copies and
    // meets the barrier.  (Not at head_dim 64, where the second bound does not fit the scalar
    // registers.)
    constexpr bool kSkip = QS > 1 && D >= 128;
    const int wrow0 = unit * UR + sub * kPT;
    const int wlast = first + min(wrow0 + kPT, L) - 1;
    const int kfull = !kSkip ? ntiles : wrow0 < L && wlast >= 0 ? min(ntiles, wlast / kPT + 1) : 0;
    if (ntiles > 0) issue(0);
    for (int kt = 0; kt < kfull; ++kt) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's copies of tile kt
      tile_barrier();                                   // ... and every wave's
      if (kt + 1 < ntiles) issue(kt + 1);               // the buffer tile kt - 1 used
      const float* kt_lds = k_lds[kt & 1];
      const float* vt_lds = v_lds[kt & 1];

      // S^T = K Q^T over d: steps (c, e).
      f32x16 st = f32x16{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float2 kv = *reinterpret_cast<const float2*>(kt_lds + (c * kPT + qi) * 4 + 2 * h);
        st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qr[c][0], st, 0, 0, 0);
        st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qr[c][1], st, 0, 0, 0);
      }
      // Mask, tile maximum, online softmax (log2 units).
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kt * kPT + 8 * j + 4 * h + r;
          if (!row_ok || key > qpos || key >= nkeys) st[4 * j + r] = -INFINITY;
          mx = fmaxf(mx, st[4 * j + r]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m, mx);
      const float alpha = mn == -INFINITY ? 1.f : exp2f(m - mn);
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = mn == -INFINITY ? 0.f : exp2f(st[e] - mn);
        st[e] = pe;
        ps += pe;
      }
      lsum = lsum * alpha + ps;
      m = mn;
#pragma unroll
      for (int b = 0; b < NDB; ++b) o[b] *= alpha;
      // O^T += V^T P^T over the tile's keys: steps (j, r).
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* vrow = vt_lds + (8 * j + 4 * h + r) * D + qi;
#pragma unroll
          for (int b = 0; b < NDB; ++b) {
            o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * b], st[4 * j + r], o[b], 0, 0, 0);
          }
        }
    }
    if constexpr (kSkip) {
      for (int kt = kfull; kt < ntiles; ++kt) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        tile_barrier();
        if (kt + 1 < ntiles) issue(kt + 1);
      }
    }
    // The two halves of a query's row sum; rows without keys (or past the sequence) give 0.
    const float ltot = lsum + __shfl_xor(lsum, 32, 64);
    const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
    if (row_ok) {
      float* op = out + ((int64_t)(row0 + myrow) * a.num_heads + head) * D;
#pragma unroll
      for (int b = 0; b < NDB; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = 32 * b + 8 * j + 4 * h;
          *reinterpret_cast<float4*>(op + d) =
              make_float4(o[b][4 * j] * inv, o[b][4 * j + 1] * inv, o[b][4 * j + 2] * inv, o[b][4 * j + 3] * inv);
        }
    }
    __syncthreads();  // every wave is done with the LDS tiles before the next unit's copies
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
                max_blocks_per_seq, num_seqs, num_tokens, 0, 0, stride, 0, 0};
  int bs_shift = -1;  // block_size = 16 << bs_shift on the MFMA path
  for (int j = 0; j <= 4; ++j)
    if (block_size == (kBlk << j)) bs_shift = j;
  hipStream_t s = as_stream(stream);
  const int eb = dtype_bytes(dtype);
  // The MFMA tile kernel: bf16 / f16, head_dim 64 / 128 / 256, block 16 << j (j <= 4), any GQA ratio G: a
  // workgroup takes GW heads of one kv-head on 4 / GW subtiles of 32 rows, GW = 4 when 4
  // divides G, else 2 when 2 does (G = 6: three workgroups of two heads per kv-head), else 1
  // (G = 3, 5, 7: one head per workgroup, the G workgroups of a kv-head share its K/V tiles in
  // the L2 of their die).
  const int G = num_heads / num_kv_heads;
  const int GW = G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
  if ((dtype == RG_DTYPE_BF16 || dtype == RG_DTYPE_F16) && scale > 0.f &&
      bs_shift >= 0 && stride % (kBlk * head_dim) == 0 && stride / (kBlk * head_dim) < (1 << 28) &&
      (head_dim == 64 || head_dim == 128 || head_dim == 256) && max_blocks_per_seq > 0 && aligned16(query) &&
      aligned16(key_cache) && aligned16(value_cache) && (stride * eb) % 16 == 0 &&
      stride * eb <= (int64_t)UINT32_MAX && aligned16(output)) {
    a.kv_stride_bytes = (uint32_t)(stride * eb);
    a.win_param = (uint32_t)(stride / (kBlk * head_dim)) << 3 | (uint32_t)bs_shift;
    const int64_t UR = (int64_t)kPT * (kPWaves / GW);  // rows per unit
    // Units per sequence from max_query_len (a hint: the kernel's last rank covers any units
    // beyond it; no query run is longer than num_tokens).
    const int64_t qmax = std::min<int64_t>(std::max<int32_t>(max_query_len, 1), num_tokens);
    a.rank_tiles = (int32_t)((qmax + UR - 1) / UR);
    // Work keys are at most ceil(prior / UR) + ceil(L / UR) <= (max(table, L) + 2 UR - 2) / UR
    // with prior + L <= the table's tokens and L <= num_tokens.
    const int64_t kbound =
        (std::max<int64_t>((int64_t)max_blocks_per_seq * block_size, num_tokens) + 2 * UR - 2) / UR + 1;
    a.sched_kbound = (kbound <= kSchedKeys && num_seqs <= kSchedSeqs) ? (int32_t)kbound : 0;
    // RG_PF_WG_PER_CU resident workgroups per CU (one at head_dim 256), split evenly over the
    // head groups, at most one per item.
    const int64_t ngroups = num_heads / GW;
    const int64_t items = (int64_t)a.rank_tiles * num_seqs;
    const int64_t wg_per_cu = head_dim > 128 ? pf_wg_per_cu<256>() : pf_wg_per_cu<128>();
    const int64_t per_group =
        std::min<int64_t>(items, std::max<int64_t>(1, wg_per_cu * device_cu_count() / ngroups));
    const dim3 grid((unsigned)(per_group * ngroups));
    // Columns: every CU holds three workgroups of one head group (workgroup b shares its CU with
    // b +- cu_count, measured), i.e. the group's workgroups q, q + C, q + 2C with C = cu / groups.
    const int64_t cus = device_cu_count();
    if (RG_PF_WEIGHTED && wg_per_cu == 3 && a.sched_kbound > 0 && cus % ngroups == 0 &&
        per_group == 3 * (cus / ngroups)) {
      a.sched_cols = (int32_t)(cus / ngroups);
    }
    auto go = [&](auto tag, auto dtag, auto gtag) {
      using T = decltype(tag);
      constexpr int D = decltype(dtag)::value;
      constexpr int W = decltype(gtag)::value;
      hipLaunchKernelGGL((prefill_mfma_kernel<T, D, W>), grid, dim3(kPThreads), 0, s, a,
                         static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key_cache),
                         static_cast<const uint16_t*>(value_cache), block_table, context_lens, cu_seqlens);
    };
    auto go_gw = [&](auto tag, auto dtag) {
      if (GW == 4) go(tag, dtag, std::integral_constant<int, 4>{});
      else if (GW == 2) go(tag, dtag, std::integral_constant<int, 2>{});
      else go(tag, dtag, std::integral_constant<int, 1>{});
    };
    using D64 = std::integral_constant<int, 64>;
    using D128 = std::integral_constant<int, 128>;
    using D256 = std::integral_constant<int, 256>;
    if (dtype == RG_DTYPE_BF16) {
      if (head_dim == 256) go_gw(bf16_t{}, D256{});
      else if (head_dim == 128) go_gw(bf16_t{}, D128{});
      else go_gw(bf16_t{}, D64{});
    } else {
      if (head_dim == 256) go_gw(f16_t{}, D256{});
      else if (head_dim == 128) go_gw(f16_t{}, D128{});
      else go_gw(f16_t{}, D64{});
    }
    return check_launch(op);
  }
  // The fp32 MFMA tile kernel: head_dim 64 / 128 / 256, any GQA ratio (GW as above), any block
  // size, 16-byte aligned rows (at head_dim 256 one workgroup per CU: 128 KB of K/V buffers).
  if (dtype == RG_DTYPE_F32 && (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
      max_blocks_per_seq > 0 && num_seqs <= 65535 && aligned16(query) && aligned16(key_cache) &&
      aligned16(value_cache) && aligned16(output) && stride % 4 == 0) {
    const int64_t UR = (int64_t)kPT * (kPWaves / GW);
    const int64_t qmax = std::min<int64_t>(std::max<int32_t>(max_query_len, 1), num_tokens);
    const dim3 grid((unsigned)((qmax + UR - 1) / UR), (unsigned)num_seqs, (unsigned)(num_heads / GW));
    auto go = [&](auto dtag, auto gtag) {
      constexpr int D = decltype(dtag)::value;
      constexpr int W = decltype(gtag)::value;
      hipLaunchKernelGGL((prefill_f32_kernel<D, W>), grid, dim3(kPThreads), 0, s, a);
    };
    auto go_gw = [&](auto dtag) {
      if (GW == 4) go(dtag, std::integral_constant<int, 4>{});
      else if (GW == 2) go(dtag, std::integral_constant<int, 2>{});
      else go(dtag, std::integral_constant<int, 1>{});
    };
    if (head_dim == 256) go_gw(std::integral_constant<int, 256>{});
    else if (head_dim == 128) go_gw(std::integral_constant<int, 128>{});
    else go_gw(std::integral_constant<int, 64>{});
    return check_launch(op);
  }
  return dispatch_dtype(dtype, [&](auto tag) {
    hipLaunchKernelGGL(prefill_generic_kernel<decltype(tag)>, dim3(num_tokens, num_heads), dim3(64),
                       0, s, a);
    return check_launch(op);
  });
}
