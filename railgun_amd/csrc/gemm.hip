// Skinny GEMM of a decode step's projections: C[M, N] = X[M, K] . W[N, K]^T with M <= 128
// (one row per decode token), bf16 / fp16 operands, fp32 accumulation, one rounding of each
// output to the operand type — candle's Linear::forward on a [tokens, in] activation
// (crates/vllm-models/src/llama/architecture.rs:38-59, 80-84; attention.rs:104-133).
//
// At M = 128 these GEMMs stream their weights once and are HBM-bound (128 flops per weight
// byte against the chip's ~310): the kernel is shaped for the weight stream.
//
// * v_mfma_f32_16x16x32 with W as the A operand (16 output columns n) and X^T as the B operand
//   (16 rows m): lane (r = lane % 16, g = lane / 16) takes W[n0 + r][k + 8g .. +8] and
//   X[m0 + r][k + 8g .. +8] from LDS.
// * Both operands reach LDS by direct global->LDS copies of 256-byte row pieces (chunks of 128
//   k), RG_GEMM_AHEAD chunks ahead of the MFMAs.  Copies of whole row pieces stream several
//   times faster per CU than 16-row x 64-byte register loads in the MFMA layout, which matters
//   for X: every workgroup reads all of it (at most 128 x K) from L2.
// * A workgroup is 4 waves over a tile of 16 MB rows x 16 NB columns (gemm_plan picks MB, NB,
//   the row tiles and splits of K per shape from a cost model of the per-CU operand stream); the
//   waves take one k-step of 32 each from every chunk and hold all NB x MB fragments of their
//   steps.  The four partial sums are added through LDS in a fixed order, so the result is
//   deterministic (graph replays reproduce eager runs bit for bit).
// * Layers with many columns (the LM head) take wide_gemm_kernel instead: the 4 waves split a
//   256-column tile rather than K, against one copy of X per workgroup.
#include <math.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "rg_common.hpp"

namespace rg {
namespace {

typedef __bf16 gbf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 gf16x8_t __attribute__((ext_vector_type(8)));
typedef float gf32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct gemm_mfma;
template <> struct gemm_mfma<bf16_t> {
  __device__ static __forceinline__ gf32x4_t run(uint4 a, uint4 b, gf32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gbf16x8_t, a),
                                                   __builtin_bit_cast(gbf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct gemm_mfma<f16_t> {
  __device__ static __forceinline__ gf32x4_t run(uint4 a, uint4 b, gf32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(gf16x8_t, a),
                                                  __builtin_bit_cast(gf16x8_t, b), c, 0, 0, 0);
  }
};

constexpr int kGemmWaves = 4;
constexpr int kGemmMaxRows = 128;
#ifndef RG_GEMM_AHEAD
#define RG_GEMM_AHEAD 2
#endif

struct GemmArgs {
  const uint16_t* x;
  const uint16_t* w;
  uint16_t* c;
  float* part;            // [splits][M][N] fp32 partial products when K is split
  int32_t M, N, K;
  int64_t ldx, ldw, ldc;  // elements between consecutive rows
  int32_t mtiles;         // row tiles of 16 MB rows (1: one tile holds every row)
  int32_t xcd_map;        // 1: the row tiles of a column tile run on one XCD (see the kernel)
  // kEpiRope: the q / k / v heads of a fused qkv projection (one head per column tile).
  const float* cos_sin;     // [positions, D]: cos at [i], sin at [D / 2 + i]
  const int32_t* positions; // [M]
  const int32_t* slots;     // [M]; negative: a padding token, not cached
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kv_stride;        // elements between cache blocks
  int32_t num_heads, num_kv_heads, block_size;
  // NORM kernels: X rows are RMS-normalised with this weight [K] (see the kernel).
  const uint16_t* norm_w;
  float norm_eps;
  int32_t stagger;  // 1: workgroups start their K loop at staggered chunks (see the kernel)
};

// Weights from this size on run with staggered chunk order: measured at the Llama-3.2-1B
// projections (paired runs, 128 / 1 rows), gate/up (67 MB) -6.5 / -16 %, the LM head (525 MB)
// -3.5 / -5.5 %, down (34 MB) -1.4 / -5 %, while qkv (12.6 MB) and o_proj (8.4 MB) were 1-4 %
// slower staggered.
#ifndef RG_GEMM_STAGGER_MIN_BYTES
#define RG_GEMM_STAGGER_MIN_BYTES (16ll << 20)
#endif
int32_t stagger_for(int32_t N, int32_t K) { return (int64_t)N * K * 2 >= RG_GEMM_STAGGER_MIN_BYTES ? 1 : 0; }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate (6 bits: [3:0] and [15:14])");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// Chunks of 128 k: 256 bytes of every row of X and W.
constexpr int kChunkK = 128;
constexpr int kChunkBytes = 2 * kChunkK;
constexpr int kLdsBytes = 160 * 1024;
constexpr int kGemmThreads = 64 * kGemmWaves;

// LDS ring of one instantiation: a slot holds a chunk of X (16 MB rows) then of W (16 NB rows).
template <int NB, int MB, int RESERVE = 0>
struct GemmRing {
  static constexpr int SLOT = 16 * (MB + NB) * kChunkBytes;
  static constexpr int FIT = (kLdsBytes - RESERVE) / SLOT;
  // AHEAD chunks in flight; with AHEAD + 2 slots the slot a wave refills was read two chunks ago,
  // so one barrier per chunk orders it; with AHEAD + 1 a second barrier follows the MFMAs.  One
  // barrier is worth more than the second chunk in flight: a ring of three slots runs one chunk
  // ahead (gate/up at 128 rows, 48 KB slots: 0.95 with SiLU·mul, with or without the folded norm,
  // in paired runs against two ahead with two barriers), larger rings RG_GEMM_AHEAD.
  static constexpr int AHEAD = FIT >= RG_GEMM_AHEAD + 2 ? RG_GEMM_AHEAD : FIT >= 3 ? FIT - 2 : FIT - 1;
  static constexpr int SLOTS = FIT >= AHEAD + 2 ? AHEAD + 2 : AHEAD + 1;
  static constexpr bool TWO_BARRIERS = SLOTS == AHEAD + 1;
  static constexpr int PER = MB + NB;  // copies per wave per chunk (1 KB each: 4 rows x 256 B)
  static constexpr int RED = NB * MB * kGemmWaves * 1024;  // every wave's partial of every fragment
  static constexpr int BYTES = SLOTS * SLOT > RED ? SLOTS * SLOT : RED;
  static_assert(AHEAD >= 1 && AHEAD * PER < 64 && BYTES + RESERVE <= kLdsBytes, "ring does not fit");
};

// NB: 16-column n-blocks per workgroup, MB: 16-row blocks of X per row tile.  blockIdx.x is
// a (column tile, row tile) pair: with xcd_map the a.mtiles row tiles of one column tile take
// consecutive slots of one XCD (workgroup b runs on XCD b % 8), so that their W tile comes from
// HBM once and from that XCD's L2 after.  blockIdx.y selects a split of K (chunks
// [y C / S, (y + 1) C / S) of the C chunks); with S > 1 the workgroup writes its fp32 partial
// tile to a.part[y] and splitk_reduce_kernel finishes.
//
// X and W reach LDS by direct copies of whole 256-byte row pieces (1 KB per wave instruction:
// 4 rows; W's copies non-temporal: each weight byte is read once per call); 16-byte piece p of row R sits at piece p ^ (R % 16), so the MFMA fragment reads
// below (16 rows at one piece) touch every bank once.  The 4 waves take one k-step of 32
// each from every chunk, so the workgroup reads each operand byte once, and each X fragment
// feeds NB MFMAs.  The quarters are summed through LDS in a fixed order.
//
// EPI = kEpiSiluMul: W holds the gate and up projections interleaved in 16-row blocks (rows
// 32j .. 32j + 15 are gate rows 16j .., rows 32j + 16 .. 32j + 31 up rows 16j ..), so n-blocks
// 2j and 2j + 1 of a tile are the gate and up columns of the same 16 outputs; the wave owning
// both writes a.c[m][16j + ..] = round(round(silu(g)) * u) from the rounded g and u (what
// silu_mul_kernel computes from a gate/up GEMM's output), a.c being [M, N / 2].
//
// EPI = kEpiRope: W is a fused q / k / v projection whose column tiles are whole heads (16 NB =
// head_dim), so n-blocks i and i + NB / 2 hold the rotation pairs (d, d + D / 2).  The wave
// owning both rounds them as the projection's output is rounded, rotates q and k heads by
// cos_sin[position] (RoPE in rotate_half form, the arithmetic of rope_cache_kernel), and writes
// q heads to a.c ([M, H, D]: a.ldc between tokens) and k / v heads into the paged caches at
// the token's slot.
constexpr int kEpiPlain = 0;
constexpr int kEpiSiluMul = 1;
constexpr int kEpiRope = 2;
constexpr int kEpiResidual = 3;  // C[m][n] <- round(C[m][n] + round(X . W^T)): the residual add
// Largest K of the NORM kernels (their norm weight is staged whole in LDS).
constexpr int kNormMaxK = 8192;

// The 8 values of a 16-byte fragment as floats.
template <typename T>
__device__ __forceinline__ void unpack8(uint4 u, float* f) {
  const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = elem<T>::to_f32((uint16_t)(wd[i] & 0xffffu));
    f[2 * i + 1] = elem<T>::to_f32((uint16_t)(wd[i] >> 16));
  }
}

// round(v[e] * f[e]) for the 8 values of a fragment.
template <typename T>
__device__ __forceinline__ uint4 scale8(uint4 u, const float* f) {
  float v[8];
  unpack8<T>(u, v);
  return make_uint4(pack2<T>(v[0] * f[0], v[1] * f[1]), pack2<T>(v[2] * f[2], v[3] * f[3]),
                    pack2<T>(v[4] * f[4], v[5] * f[5]), pack2<T>(v[6] * f[6], v[7] * f[7]));
}

// acc + the sum of the squares of a fragment's 8 values (four dot2 steps, fp32 accumulation).
template <typename T> __device__ __forceinline__ float sum_squares8(uint4 u, float acc);
template <> __device__ __forceinline__ float sum_squares8<bf16_t>(uint4 u, float acc) {
  const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wd[i]), __builtin_bit_cast(bf16x2_t, wd[i]),
                                          acc, false);
  }
  return acc;
}
template <> __device__ __forceinline__ float sum_squares8<f16_t>(uint4 u, float acc) {
  const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, wd[i]), __builtin_bit_cast(f16x2_t, wd[i]), acc, false);
  }
  return acc;
}

// Four stored values plus round(v): round(c + round(v)) per value (the residual add of
// rms_norm_kernel on a rounded projection output).
template <typename T>
__device__ __forceinline__ uint2 add_rounded(uint2 c, gf32x4_t v) {
  const float c0 = elem<T>::to_f32((uint16_t)(c.x & 0xffffu)), c1 = elem<T>::to_f32((uint16_t)(c.x >> 16));
  const float c2 = elem<T>::to_f32((uint16_t)(c.y & 0xffffu)), c3 = elem<T>::to_f32((uint16_t)(c.y >> 16));
  auto rnd = [](float x) { return std::is_same<T, bf16_t>::value ? (float)(__bf16)x : (float)(_Float16)x; };
  return make_uint2(pack2<T>(c0 + rnd(v[0]), c1 + rnd(v[1])), pack2<T>(c2 + rnd(v[2]), c3 + rnd(v[3])));
}

template <typename T, int NB, int MB, int EPI, bool NORM = false>
__global__ __launch_bounds__(kGemmThreads) void skinny_gemm_kernel(GemmArgs a) {
  static_assert(EPI == kEpiPlain || EPI == kEpiResidual || NB % 2 == 0,
                "gate/up and rotation pairs need an even number of n-blocks");
  using MF = gemm_mfma<T>;
  constexpr int NORM_BYTES = NORM ? 2 * kNormMaxK : 0;
  using RG = GemmRing<NB, MB, NORM_BYTES>;
  constexpr int KS = kGemmWaves;
  constexpr int D = RG::AHEAD;
  static_assert(RG::BYTES + NORM_BYTES <= kLdsBytes, "norm weight does not fit");
  // Wave 0 has up to 2 kNormMaxK / 1024 norm-weight copies in flight with its first chunks.
  static_assert(!NORM || D * RG::PER + 2 * kNormMaxK / 1024 < 64, "vmcnt range");
  __shared__ __attribute__((aligned(16))) char lds[RG::BYTES + NORM_BYTES];
  const uint32_t lds_base = (uint32_t)(uintptr_t)((RG_LDS char*)lds);

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int total = a.K / kChunkK;
  const int cb = (int)((int64_t)blockIdx.y * total / gridDim.y);
  const int chunks = (int)((int64_t)(blockIdx.y + 1) * total / gridDim.y) - cb;
  int nt = blockIdx.x, mt = 0;
  if (a.mtiles > 1) {
    if (a.xcd_map) {
      const int k = blockIdx.x >> 3;
      mt = k % a.mtiles;
      nt = (k / a.mtiles) * 8 + (blockIdx.x & 7);
    } else {
      mt = blockIdx.x % a.mtiles;
      nt = blockIdx.x / a.mtiles;
    }
  }
  const int n0 = nt * NB * 16;
  const int m0 = mt * 16 * MB;
  const int mrows = min(16 * MB, a.M - m0);  // rows of this tile

  // Copy sources: instruction q of wave w moves rows 4 (w * MB + q) .. +3 of X (then rows
  // 4 (w * NB + q) .. +3 of W), lane (row 4q' + lane / 16, piece (lane % 16) ^ (row % 16)).
  const char* xbase = reinterpret_cast<const char*>(a.x + (int64_t)m0 * a.ldx) + (int64_t)cb * kChunkBytes;
  const char* wbase = reinterpret_cast<const char*>(a.w + (int64_t)n0 * a.ldw) + (int64_t)cb * kChunkBytes;
  uint32_t xoff[MB], woff[NB];
#pragma unroll
  for (int q = 0; q < MB; ++q) {
    const int row = 4 * (w * MB + q) + (lane >> 4);
    xoff[q] = (uint32_t)(min(row, mrows - 1) * a.ldx * 2 + (((lane & 15) ^ (row & 15)) << 4));
  }
#pragma unroll
  for (int q = 0; q < NB; ++q) {
    const int row = 4 * (w * NB + q) + (lane >> 4);
    woff[q] = (uint32_t)(row * a.ldw * 2 + (((lane & 15) ^ (row & 15)) << 4));
  }
  // With a.stagger, loop position c reads chunk (c + rot) mod chunks, rot = the workgroup's
  // position among those of its die (workgroup b runs on XCD b mod 8): the workgroups of a die
  // start at different chunks instead of all reading chunk c of their rows at once (X and W
  // rows are K * 2 bytes apart, so chunk c of every row tends to fall in the same L2 channel).
  const int rot = a.stagger && chunks > 0 ? (int)((blockIdx.x >> 3) % (unsigned)chunks) : 0;
  auto chunk_of = [&](int c) __attribute__((always_inline)) {
    const int cc = c + rot;
    return cc >= chunks ? cc - chunks : cc;
  };
  auto issue = [&](int c) __attribute__((always_inline)) {
    const uint32_t slot = lds_base + (uint32_t)((c % RG::SLOTS) * RG::SLOT);
    const int64_t kb = (int64_t)chunk_of(c) * kChunkBytes;
#pragma unroll
    for (int q = 0; q < MB; ++q) lds_dma16_s(xbase + kb, xoff[q], slot + (w * MB + q) * 1024);
#pragma unroll
    for (int q = 0; q < NB; ++q) lds_dma16_s_nt(wbase + kb, woff[q], slot + 16 * MB * kChunkBytes + (w * NB + q) * 1024);
  };

  gf32x4_t acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[i][mb] = gf32x4_t{0.f, 0.f, 0.f, 0.f};

  // NORM: wave 0 copies the norm weight into LDS ahead of its first chunk, so the first chunk's
  // wait covers it (copies complete in issue order for the counter).
  if constexpr (NORM) {
    if (w == 0) {
      const uint32_t nbytes = (uint32_t)a.K * 2;
      for (uint32_t q = 0; q * 1024 < nbytes; ++q) {
        lds_dma16_s(reinterpret_cast<const char*>(a.norm_w), min(q * 1024 + (uint32_t)lane * 16, nbytes - 16),
                    lds_base + (uint32_t)RG::BYTES + q * 1024);
      }
    }
  }
  float ss[MB];  // NORM: this lane's part of the sum of squares of row 16 mb + r
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) ss[mb] = 0.f;

  // Fragment reads: row R of the slot's X (or W) rows, piece 4w + g of the chunk.
  const int piece = ((4 * w + g) ^ r) << 4;
  for (int c = 0; c < D && c < chunks; ++c) issue(c);
  for (int c = 0; c < chunks; ++c) {
    if (c + D < chunks) issue(c + D);
    // Wait until at most min(D, chunks - 1 - c) chunks of this wave's copies are in flight.
    const int ahead = min(D, chunks - 1 - c);
    [&]<int... J>(std::integer_sequence<int, J...>) __attribute__((always_inline)) {
      ((ahead == J ? wait_vmcnt<J * RG::PER>() : void()), ...);
    }(std::make_integer_sequence<int, D + 1>{});
    tile_barrier();
    const char* slot = lds + (c % RG::SLOTS) * RG::SLOT;
    uint4 wv[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      wv[i] = *reinterpret_cast<const uint4*>(slot + (16 * MB + 16 * i + r) * kChunkBytes + piece);
    }
    // NORM: the MFMA takes x and W with one of them scaled by the norm weight of its k and
    // rounded — W when the tile has fewer W fragments than X fragments, else x — and the row
    // scale 1 / rms(x) is applied to the sums at the end.  fp16 always scales W: x is the
    // residual stream, not yet divided by its rms, and x * w_norm can pass fp16's 65504 (inf,
    // then NaN logits) where the normalised operand of the unfused chain is about 1 in size;
    // bf16 has fp32's exponent range and takes the cheaper side.
    constexpr bool SCALE_W = NB < MB || std::is_same<T, f16_t>::value;
    float nw[8];  // the norm weight of this lane's 8 k
    if constexpr (NORM) {
      const uint4 u = *reinterpret_cast<const uint4*>(lds + RG::BYTES + (cb + chunk_of(c)) * kChunkBytes + (4 * w + g) * 16);
      unpack8<T>(u, nw);
      if constexpr (SCALE_W) {
#pragma unroll
        for (int i = 0; i < NB; ++i) wv[i] = scale8<T>(wv[i], nw);
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      uint4 xv = *reinterpret_cast<const uint4*>(slot + (16 * mb + r) * kChunkBytes + piece);
      if constexpr (NORM) {
        ss[mb] = sum_squares8<T>(xv, ss[mb]);
        if constexpr (!SCALE_W) xv = scale8<T>(xv, nw);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) acc[i][mb] = MF::run(wv[i], xv, acc[i][mb]);
    }
    if constexpr (RG::TWO_BARRIERS) tile_barrier();
  }

  // Every wave leaves its partial of every fragment f = i * MB + mb at red[f][w]; then wave w
  // finishes output items w, w + 4, ... (fragments, or the gate / up and rotation pairs of
  // fragments for kEpiSiluMul and kEpiRope), summing the four partials in wave order.  A wave's
  // items are independent, so the unrolled loop overlaps one item's LDS reads with another's
  // arithmetic (the wave is alone on its SIMD here).  Every copy has landed (the last wait was
  // for 0).
  tile_barrier();
  gf32x4_t* red = reinterpret_cast<gf32x4_t*>(lds);
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) red[((i * MB + mb) * KS + w) * 64 + lane] = acc[i][mb];
  // NORM: the row sums of squares, over the 4 lanes of a row (k pieces g), then over the waves
  // (k-steps w) through the norm weight's LDS, which no wave reads any more.
  float* sq = reinterpret_cast<float*>(lds + RG::BYTES);
  if constexpr (NORM) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      ss[mb] += __shfl_xor(ss[mb], 16);
      ss[mb] += __shfl_xor(ss[mb], 32);
      if (g == 0) sq[(w * MB + mb) * 16 + r] = ss[mb];
    }
  }
  __syncthreads();
  float rs[MB];  // NORM: 1 / rms of row 16 mb + r
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    rs[mb] = 1.f;
    if constexpr (NORM) {
      float t = sq[mb * 16 + r];
#pragma unroll
      for (int j = 1; j < KS; ++j) t += sq[(j * MB + mb) * 16 + r];
      rs[mb] = rsqrtf(t / (float)a.K + a.norm_eps);
    }
  }
  auto partial_sum = [&](int f) __attribute__((always_inline)) {
    gf32x4_t v = red[(f * KS) * 64 + lane];
#pragma unroll
    for (int j = 1; j < KS; ++j) v += red[(f * KS + j) * 64 + lane];
    if constexpr (NORM) v *= rs[f % MB];
    return v;
  };
  auto round_to = [](float v) __attribute__((always_inline)) {
    return std::is_same<T, bf16_t>::value ? (float)(__bf16)v : (float)(_Float16)v;
  };
  constexpr int ITEMS = EPI == kEpiPlain || EPI == kEpiResidual ? NB * MB : (NB / 2) * MB;
  constexpr int PER_WAVE = (ITEMS + KS - 1) / KS;

  if constexpr (EPI == kEpiRope) {
    constexpr int HD = 8 * NB;  // half the head
    const int hg = n0 / (16 * NB);  // head among the H q, H_kv k and H_kv v heads
    const bool is_q = hg < a.num_heads, is_v = hg >= a.num_heads + a.num_kv_heads;
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int q = w + KS * j;
      if (q >= ITEMS) break;
      const int p = q / MB, mb = q % MB;
      if (16 * mb + r >= mrows) continue;
      const gf32x4_t vl = partial_sum(p * MB + mb), vh = partial_sum((p + NB / 2) * MB + mb);
      const int m = m0 + 16 * mb + r;
      const int d = 16 * p + 4 * g;  // this lane's columns d .. d + 3 and HD + d ..
      float ol[4], oh[4];
      if (is_v) {
#pragma unroll
        for (int e = 0; e < 4; ++e) ol[e] = vl[e], oh[e] = vh[e];
      } else {
        const float* cs = a.cos_sin + (int64_t)a.positions[m] * (2 * HD);
        const float4 c4 = *reinterpret_cast<const float4*>(cs + d);
        const float4 s4 = *reinterpret_cast<const float4*>(cs + HD + d);
        const float c[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) rope_rotate_pair(round_to(vl[e]), round_to(vh[e]), c[e], sn[e], ol[e], oh[e]);
      }
      uint16_t* dst;
      if (is_q) {
        dst = a.c + (int64_t)m * a.ldc + (int64_t)hg * (2 * HD);
      } else {
        const int32_t slot = a.slots[m];
        if (slot < 0) continue;  // padding token
        const int kvh = is_v ? hg - a.num_heads - a.num_kv_heads : hg - a.num_heads;
        dst = (is_v ? a.v_cache : a.k_cache) + (int64_t)(slot / a.block_size) * a.kv_stride +
              ((int64_t)kvh * a.block_size + slot % a.block_size) * (2 * HD);
      }
      *reinterpret_cast<uint2*>(dst + d) = make_uint2(pack2<T>(ol[0], ol[1]), pack2<T>(ol[2], ol[3]));
      *reinterpret_cast<uint2*>(dst + HD + d) = make_uint2(pack2<T>(oh[0], oh[1]), pack2<T>(oh[2], oh[3]));
    }
    return;
  }

  if constexpr (EPI == kEpiSiluMul) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int q = w + KS * j;
      if (q >= ITEMS) break;
      const int jp = q / MB, mb = q % MB;
      if (16 * mb + r >= mrows) continue;
      const gf32x4_t vg = partial_sum(2 * jp * MB + mb), vu = partial_sum((2 * jp + 1) * MB + mb);
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float gv = round_to(vg[e]);
        o[e] = round_to(gv / (1.f + expf(-gv))) * round_to(vu[e]);
      }
      const int n = (n0 / 32 + jp) * 16 + 4 * g;
      *reinterpret_cast<uint2*>(a.c + (int64_t)(m0 + 16 * mb + r) * a.ldc + n) =
          make_uint2(pack2<T>(o[0], o[1]), pack2<T>(o[2], o[3]));
    }
    return;
  }

  // Lane (r, g) holds C[m0 + 16 mb + r][n0 + 16 i + 4g .. +3].
#pragma unroll
  for (int j = 0; j < PER_WAVE; ++j) {
    const int f = w + KS * j;
    if (f >= ITEMS) break;
    const int i = f / MB, mb = f % MB;
    if (16 * mb + r >= mrows) continue;
    const gf32x4_t v = partial_sum(f);
    const int m = m0 + 16 * mb + r;
    const int n = n0 + 16 * i + 4 * g;
    if (gridDim.y > 1) {
      *reinterpret_cast<gf32x4_t*>(a.part + ((int64_t)blockIdx.y * a.M + m) * a.N + n) = v;
    } else {
      uint2* dst = reinterpret_cast<uint2*>(a.c + (int64_t)m * a.ldc + n);
      if constexpr (EPI == kEpiResidual) *dst = add_rounded<T>(*dst, v);
      else *dst = make_uint2(pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]));
    }
  }
}

// Wide form for layers with many output columns (the LM head: 128k columns): the 4 waves split
// the tile's columns instead of K, NW 16-column blocks each, so a workgroup covers 64 NW columns
// against one copy of X in LDS and X's bytes per weight byte drop from 2 (128 rows against 64
// columns) to 128 / (64 NW).  Chunks are 64 k (128-byte row pieces, 16-byte piece p of row R at
// piece p ^ (R % 8)) so that the ring holds several chunks ahead; each wave reads every X
// fragment and its own W fragments, and holds only its columns' sums: no reduction between the
// waves, each writes its columns.  Plain or residual epilogue (EPI), one pass over K.
constexpr int kWideK = 64;
constexpr int kWideRow = 2 * kWideK;  // bytes of a row piece
template <int NW, int MB>
struct WideRing {
  static constexpr int ROWS = 16 * MB + 16 * NW * kGemmWaves;  // X rows, then W rows
  static constexpr int SLOT = ROWS * kWideRow;
  static constexpr int FIT = kLdsBytes / SLOT;
  // One barrier per chunk where the ring allows it, as in GemmRing (128 rows, three 48 KB slots:
  // one chunk ahead 0.986 against two ahead with two barriers; 64 rows 0.978).
  static constexpr int AHEAD = FIT >= 5 ? 3 : FIT >= 3 ? FIT - 2 : FIT - 1;
  static constexpr int SLOTS = FIT >= AHEAD + 2 ? AHEAD + 2 : AHEAD + 1;
  static constexpr bool TWO_BARRIERS = SLOTS == AHEAD + 1;
  static constexpr int QX = 16 * MB / 8 / kGemmWaves;  // X copies per wave per chunk (1 KB: 8 rows)
  static constexpr int QW = 2 * NW;                    // W copies per wave per chunk
  static constexpr int PER = QX + QW;
  static_assert(QX * 8 * kGemmWaves == 16 * MB, "X rows per wave");
  static_assert(AHEAD >= 1 && AHEAD * PER < 64 && SLOTS * SLOT <= kLdsBytes, "wide ring does not fit");
};
template <typename T, int NW, int MB, int EPI>
__global__ __launch_bounds__(kGemmThreads) void wide_gemm_kernel(GemmArgs a) {
  static_assert(EPI == kEpiPlain || EPI == kEpiResidual, "plain or residual epilogue");
  using MF = gemm_mfma<T>;
  using RG = WideRing<NW, MB>;
  constexpr int D = RG::AHEAD;
  __shared__ __attribute__((aligned(16))) char lds[RG::SLOTS * RG::SLOT];
  const uint32_t lds_base = (uint32_t)(uintptr_t)((RG_LDS char*)lds);
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int chunks = a.K / kWideK;
  const int n0 = blockIdx.x * (16 * NW * kGemmWaves);
  const int mrows = min(16 * MB, a.M);

  // Copy sources: instruction q of wave w moves X rows 8 (w QX + q) .. +7 (then W rows
  // 8 (w QW + q) .. +7 of the tile), lane (row + lane / 8, piece (lane % 8) ^ (row % 8)).
  const char* xbase = reinterpret_cast<const char*>(a.x);
  const char* wbase = reinterpret_cast<const char*>(a.w + (int64_t)n0 * a.ldw);
  uint32_t xoff[RG::QX], woff[RG::QW];
#pragma unroll
  for (int q = 0; q < RG::QX; ++q) {
    const int row = 8 * (w * RG::QX + q) + (lane >> 3);
    xoff[q] = (uint32_t)(min(row, mrows - 1) * a.ldx * 2 + (((lane & 7) ^ (row & 7)) << 4));
  }
#pragma unroll
  for (int q = 0; q < RG::QW; ++q) {
    const int row = 8 * (w * RG::QW + q) + (lane >> 3);
    woff[q] = (uint32_t)(row * a.ldw * 2 + (((lane & 7) ^ (row & 7)) << 4));
  }
  // Staggered chunk order for large weights, as in skinny_gemm_kernel.
  const int rot = a.stagger && chunks > 0 ? (int)((blockIdx.x >> 3) % (unsigned)chunks) : 0;
  auto issue = [&](int c) __attribute__((always_inline)) {
    const uint32_t slot = lds_base + (uint32_t)((c % RG::SLOTS) * RG::SLOT);
    const int cc = c + rot;
    const int64_t kb = (int64_t)(cc >= chunks ? cc - chunks : cc) * kWideRow;
#pragma unroll
    for (int q = 0; q < RG::QX; ++q) lds_dma16_s(xbase + kb, xoff[q], slot + (w * RG::QX + q) * 1024);
#pragma unroll
    for (int q = 0; q < RG::QW; ++q)
      lds_dma16_s_nt(wbase + kb, woff[q], slot + 16 * MB * kWideRow + (w * RG::QW + q) * 1024);
  };

  gf32x4_t acc[NW][MB];
#pragma unroll
  for (int i = 0; i < NW; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[i][mb] = gf32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int c = 0; c < D && c < chunks; ++c) issue(c);
  for (int c = 0; c < chunks; ++c) {
    if (c + D < chunks) issue(c + D);
    const int ahead = min(D, chunks - 1 - c);
    [&]<int... J>(std::integer_sequence<int, J...>) __attribute__((always_inline)) {
      ((ahead == J ? wait_vmcnt<J * RG::PER>() : void()), ...);
    }(std::make_integer_sequence<int, D + 1>{});
    tile_barrier();
    const char* slot = lds + (c % RG::SLOTS) * RG::SLOT;
#pragma unroll
    for (int ks = 0; ks < kWideK / 32; ++ks) {
      // Lane (r, g) takes k 32 ks + 8 g .. +8 of row r of each 16-row block: piece 4 ks + g.
      const int piece = ((4 * ks + g) ^ (r & 7)) << 4;
      uint4 wv[NW];
#pragma unroll
      for (int i = 0; i < NW; ++i)
        wv[i] = *reinterpret_cast<const uint4*>(slot + (16 * MB + 16 * (w * NW + i) + r) * kWideRow + piece);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint4 xv = *reinterpret_cast<const uint4*>(slot + (16 * mb + r) * kWideRow + piece);
#pragma unroll
        for (int i = 0; i < NW; ++i) acc[i][mb] = MF::run(wv[i], xv, acc[i][mb]);
      }
    }
    if constexpr (RG::TWO_BARRIERS) tile_barrier();
  }
  // Lane (r, g) holds C[16 mb + r][n0 + 16 (w NW + i) + 4 g .. +3].
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    if (16 * mb + r >= mrows) continue;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const gf32x4_t v = acc[i][mb];
      uint2* dst = reinterpret_cast<uint2*>(a.c + (int64_t)(16 * mb + r) * a.ldc + n0 + 16 * (w * NW + i) + 4 * g);
      if constexpr (EPI == kEpiResidual) *dst = add_rounded<T>(*dst, v);
      else *dst = make_uint2(pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]));
    }
  }
}

// out[m][n] = round(sum over the S splits, in split order, of part[s][m][n]): 4 columns per lane.
// RES: out[m][n] = round(out[m][n] + round(sum)), the residual add.
template <typename T, bool RES>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs a, int S) {
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (idx >= (int64_t)a.M * a.N) return;
  const int m = (int)(idx / a.N), n = (int)(idx % a.N);
  gf32x4_t v = *reinterpret_cast<const gf32x4_t*>(a.part + idx);
  for (int s = 1; s < S; ++s) v += *reinterpret_cast<const gf32x4_t*>(a.part + (int64_t)s * a.M * a.N + idx);
  uint2* dst = reinterpret_cast<uint2*>(a.c + (int64_t)m * a.ldc + n);
  if constexpr (RES) *dst = add_rounded<T>(*dst, v);
  else *dst = make_uint2(pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]));
}

template <typename T, int NB, int EPI = kEpiPlain, bool NORM = false>
void launch_gemm_mb(const GemmArgs& a, int mb, int splits, hipStream_t s) {
  const dim3 grid((unsigned)(a.N / (16 * NB) * a.mtiles), (unsigned)splits);
  switch (mb) {
    case 1: hipLaunchKernelGGL((skinny_gemm_kernel<T, NB, 1, EPI, NORM>), grid, dim3(kGemmThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((skinny_gemm_kernel<T, NB, 2, EPI, NORM>), grid, dim3(kGemmThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((skinny_gemm_kernel<T, NB, 4, EPI, NORM>), grid, dim3(kGemmThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((skinny_gemm_kernel<T, NB, 8, EPI, NORM>), grid, dim3(kGemmThreads), 0, s, a); break;
  }
  if ((EPI == kEpiPlain || EPI == kEpiResidual) && splits > 1) {
    const int64_t quads = (int64_t)a.M * a.N / 4;
    hipLaunchKernelGGL((splitk_reduce_kernel<T, EPI == kEpiResidual>), dim3((unsigned)ceil_div(quads, 256)), dim3(256),
                       0, s, a, splits);
  }
}

// The wide form (wide_gemm_kernel) for layers of at least RG_GEMM_WIDE_MIN_N columns at more than
// RG_GEMM_WIDE_MIN_M rows, RG_GEMM_WIDE_NW 16-column blocks per wave, X tiles of 32, 64 or 128
// rows.  Measured on the Llama-3.2-1B LM head (128,256 x 2048, weights cold, paired runs):
// 128 rows 154.7 -> 112.0 us (hipBLASLt 133.7), 100 rows 153.1 -> 109.0, 64 rows 121.5 -> 99.3,
// 40 rows 110.1 -> 96.7, 32 rows 95.4 -> 89.0, 24 rows 94.3 -> 90.2, 17 rows 92.7 -> 88.5, but
// 9 rows 83.4 -> 87.1; two blocks per wave (128 columns per workgroup) gave 134.9 us at 128 rows.
#ifndef RG_GEMM_WIDE_MIN_N
#define RG_GEMM_WIDE_MIN_N 32768
#endif
#ifndef RG_GEMM_WIDE_NW
#define RG_GEMM_WIDE_NW 4
#endif
#ifndef RG_GEMM_WIDE_MIN_M
#define RG_GEMM_WIDE_MIN_M 16
#endif
constexpr int kWideCols = 16 * RG_GEMM_WIDE_NW * kGemmWaves;
bool wide_fits(int M, int N, int K, int64_t ldw) {
  return RG_GEMM_WIDE_MIN_N > 0 && M > RG_GEMM_WIDE_MIN_M && N >= RG_GEMM_WIDE_MIN_N && N % kWideCols == 0 && K % kWideK == 0 &&
         (int64_t)(kWideCols - 1) * ldw * 2 + 2 * (int64_t)K <= INT32_MAX;
}
template <typename T, int EPI>
void launch_wide(const GemmArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.N / kWideCols));
  if (a.M > 64) hipLaunchKernelGGL((wide_gemm_kernel<T, RG_GEMM_WIDE_NW, 8, EPI>), grid, dim3(kGemmThreads), 0, s, a);
  else if (a.M > 32) hipLaunchKernelGGL((wide_gemm_kernel<T, RG_GEMM_WIDE_NW, 4, EPI>), grid, dim3(kGemmThreads), 0, s, a);
  else hipLaunchKernelGGL((wide_gemm_kernel<T, RG_GEMM_WIDE_NW, 2, EPI>), grid, dim3(kGemmThreads), 0, s, a);
}

template <typename T, int EPI = kEpiPlain>
void launch_gemm(const GemmArgs& a, int nb, int mb, int splits, hipStream_t s) {
  if (nb == 4) launch_gemm_mb<T, 4, EPI>(a, mb, splits, s);
  else if (nb == 2) launch_gemm_mb<T, 2, EPI>(a, mb, splits, s);
  else launch_gemm_mb<T, 1, EPI>(a, mb, splits, s);
}

template <typename T, bool NORM = false>
void launch_gemm_silu_mul(const GemmArgs& a, int nb, int mb, hipStream_t s) {
  if (nb == 4) launch_gemm_mb<T, 4, kEpiSiluMul, NORM>(a, mb, 1, s);
  else launch_gemm_mb<T, 2, kEpiSiluMul, NORM>(a, mb, 1, s);
}

template <typename T, bool NORM = false>
void launch_gemm_rope(const GemmArgs& a, int nb, int mb, hipStream_t s) {
  if (nb == 4) launch_gemm_mb<T, 4, kEpiRope, NORM>(a, mb, 1, s);
  else launch_gemm_mb<T, 2, kEpiRope, NORM>(a, mb, 1, s);
}

// LDS bytes of a workgroup of the (NB, MB) instantiation (GemmRing<NB, MB, reserve>::BYTES +
// reserve, the norm weight's bytes of the NORM kernels).
int ring_bytes(int nb, int mb, int reserve = 0) {
  const int slot = 16 * (mb + nb) * kChunkBytes;
  const int fit = (kLdsBytes - reserve) / slot;
  const int ahead = fit >= RG_GEMM_AHEAD + 2 ? RG_GEMM_AHEAD : fit >= 3 ? fit - 2 : fit - 1;
  const int slots = fit >= ahead + 2 ? ahead + 2 : ahead + 1;
  return std::max(slots * slot, nb * mb * kGemmWaves * 1024) + reserve;
}

// Workgroup shape: 16-column n-blocks (NB) and 16-row blocks (MB) per workgroup, row tiles
// ceil(M / 16 MB) and splits of K, chosen by a cost model of the per-CU operand stream
// calibrated on MI355X (a sweep of every shape at the Llama-3.2-1B projections for 1 to 128
// rows; the model's pick is the measured best or within 10 % of it):
//   workgroups = row tiles x column tiles x splits, R = CUs x resident workgroups per CU (LDS),
//   stream = 3 us x ceil(workgroups / R) + 0.047 us x ceil(workgroups / CUs) x (MB + NB) x chunks / S
//            (0.047 us per 16 rows x 128 k: 4 KB of copies),
//   weights = N K 2 B / 5.5 TB/s,
//   time = max(stream, weights) + 0.2 min(stream, weights) + (S > 1: 2 us + S M N 8 B / 3 TB/s for
//          the partials and their reduce).
// Each workgroup streams its rows of X and its columns of W once per K range; small row tiles
// cut the X bytes of narrow layers, and the XCD-aware order keeps their re-reads of W in L2.
struct GemmPlan { int nb, mb, mtiles, splits, xcd; };
GemmPlan gemm_plan(int M, int N, int K, int cus, bool pairs = false, int only_nb = 0, bool norm = false) {
  const int nblk = N / 16, chunks = K / kChunkK;
  GemmPlan best{1, 1, M, 1, 0};
  double best_t = 1e30;
  for (int mb : {1, 2, 4, 8}) {
    if (mb > 1 && 16 * (mb / 2) >= M) continue;  // a smaller row tile already holds every row
    const int mtiles = (M + 16 * mb - 1) / (16 * mb);
    for (int nb : {4, 2, 1}) {
      if (nblk % nb != 0 || (pairs && nb == 1) || (only_nb && nb != only_nb)) continue;
      const int resident = std::max(1, std::min(4, kLdsBytes / ring_bytes(nb, mb, norm ? 2 * kNormMaxK : 0)));
      for (int splits : {1, 2, 4}) {
        if (splits > 1 && (pairs || norm || chunks / splits < 8)) continue;
        const int64_t wgs = (int64_t)mtiles * (nblk / nb) * splits;
        const double stream = 3.0 * (double)ceil_div(wgs, (int64_t)cus * resident) +
                              0.047 * (double)ceil_div(wgs, cus) * (mb + nb) * (chunks / splits);
        const double weights = (double)N * K * 2 / 5.5e6;
        double t = std::max(stream, weights) + 0.2 * std::min(stream, weights);
        if (splits > 1) t += 2.0 + (double)splits * M * N * 8 / 3.0e6;
        if (t < best_t - 1e-9) {
          best_t = t;
          best = GemmPlan{nb, mb, mtiles, splits, mtiles > 1 && (nblk / nb) % 8 == 0 ? 1 : 0};
        }
      }
    }
  }
  return best;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace rg

using namespace rg;

extern "C" size_t rg_linear_workspace_bytes(int32_t num_rows, int32_t out_features, int32_t in_features) {
  if (num_rows <= 0 || num_rows > kGemmMaxRows || out_features <= 0 || out_features % 16 != 0 ||
      in_features <= 0 || in_features % kChunkK != 0) {
    return 0;
  }
  if (wide_fits(num_rows, out_features, in_features, in_features)) return 0;  // the wide form: one pass
  const GemmPlan p = gemm_plan(num_rows, out_features, in_features, device_cu_count());
  return p.splits > 1 ? (size_t)p.splits * num_rows * out_features * sizeof(float) : 0;
}

namespace rg {
namespace {
// Checks shared by the rg_linear entries (N: weight rows, out_cols: output row length).
// Returns RG_OK, or a failure status; `empty` is set for a call with nothing to do.
int check_linear(const char* op, const void* x, const void* weight, const void* out, int32_t M, int32_t N,
                 int32_t K, int32_t out_cols, int64_t ldx, int64_t ldw, int64_t ldo, int32_t dtype, bool& empty) {
  empty = false;
  if (dtype != RG_DTYPE_BF16 && dtype != RG_DTYPE_F16) {
    return fail(RG_ERR_NOT_SUPPORTED, "%s: bf16 or f16 operands only, got dtype %d", op, dtype);
  }
  if (M < 0 || N < 0 || K < 0) return fail(RG_ERR_INVALID_ARGUMENT, "%s: negative size", op);
  if (M == 0 || N == 0) {
    empty = true;
    return ok();
  }
  if (M > kGemmMaxRows || N % 16 != 0 || K % kChunkK != 0 || K == 0) {
    return fail(RG_ERR_NOT_SUPPORTED,
                "%s: needs num_rows <= %d, out_features a multiple of 16 and in_features a positive "
                "multiple of %d (got %d, %d, %d)", op, kGemmMaxRows, kChunkK, M, N, K);
  }
  if (!x || !weight || !out) return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  if (ldx < K || ldw < K || ldo < out_cols) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: a row stride is shorter than its row", op);
  }
  if (!aligned16(x) || !aligned16(weight) || ldx % 8 != 0 || ldw % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(out) & 7u) != 0 || ldo % 4 != 0) {
    return fail(RG_ERR_NOT_SUPPORTED,
                "%s: operands and row strides must be 16-byte aligned (output 8-byte aligned)", op);
  }
  // The copies address a row as a 32-bit byte offset from X (from the workgroup's first W row).
  if ((int64_t)(M - 1) * ldx * 2 + 2 * (int64_t)K > INT32_MAX || (int64_t)63 * ldw * 2 + 2 * (int64_t)K > INT32_MAX) {
    return fail(RG_ERR_NOT_SUPPORTED, "%s: row strides too large for 32-bit copy offsets", op);
  }
  return RG_OK;
}
}  // namespace
}  // namespace rg

namespace rg {
namespace {
// rg_linear (EPI kEpiPlain) and rg_linear_residual (kEpiResidual: out is the residual stream).
template <int EPI>
int linear_entry(const char* op, const void* x, const void* weight, void* out, int32_t M, int32_t N, int32_t K,
                 int64_t ldx, int64_t ldw, int64_t ldo, void* workspace, size_t workspace_bytes, int32_t dtype,
                 void* stream) {
  bool empty = false;
  if (int st = check_linear(op, x, weight, out, M, N, K, N, ldx, ldw, ldo, dtype, empty)) return st;
  if (empty) return ok();
  GemmPlan plan = gemm_plan(M, N, K, device_cu_count());
  const size_t need = plan.splits > 1 ? (size_t)plan.splits * M * N * sizeof(float) : 0;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))) {
    plan.splits = 1;  // no (or too small a) workspace: one pass over K
  }
  GemmArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
             static_cast<float*>(workspace), M, N, K, ldx, ldw, ldo, plan.mtiles, plan.xcd};
  a.stagger = stagger_for(N, K);
  hipStream_t s = as_stream(stream);
  if (wide_fits(M, N, K, ldw)) {
    if (dtype == RG_DTYPE_BF16) launch_wide<bf16_t, EPI>(a, s);
    else launch_wide<f16_t, EPI>(a, s);
    return check_launch(op);
  }
  if (dtype == RG_DTYPE_BF16) launch_gemm<bf16_t, EPI>(a, plan.nb, plan.mb, plan.splits, s);
  else launch_gemm<f16_t, EPI>(a, plan.nb, plan.mb, plan.splits, s);
  return check_launch(op);
}

// The RMSNorm weight of the NORM kernels: present, 16-byte aligned, K within the LDS copy.
int check_norm(const char* op, const void* norm_weight, int32_t K, float eps) {
  if (!norm_weight || !aligned16(norm_weight)) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: norm_weight must be a 16-byte aligned [in_features] vector", op);
  }
  if (K > kNormMaxK) return fail(RG_ERR_NOT_SUPPORTED, "%s: in_features at most %d (got %d)", op, kNormMaxK, K);
  if (!(eps >= 0.f)) return fail(RG_ERR_INVALID_ARGUMENT, "%s: eps must be non-negative", op);
  return RG_OK;
}

int silu_mul_entry(const char* op, const void* x, const void* norm_weight, float eps, const void* weight_gate_up,
                   void* out, int32_t M, int32_t I, int32_t K, int64_t ldx, int64_t ldw, int64_t ldo, int32_t dtype,
                   void* stream) {
  if (I < 0 || I % 16 != 0) {
    return fail(RG_ERR_NOT_SUPPORTED, "%s: intermediate_size must be a multiple of 16 (got %d)", op, I);
  }
  bool empty = false;
  if (int st = check_linear(op, x, weight_gate_up, out, M, 2 * I, K, I, ldx, ldw, ldo, dtype, empty)) return st;
  if (empty) return ok();
  const bool norm = norm_weight != nullptr;
  const GemmPlan plan = gemm_plan(M, 2 * I, K, device_cu_count(), true, 0, norm);
  GemmArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight_gate_up),
             static_cast<uint16_t*>(out), nullptr, M, 2 * I, K, ldx, ldw, ldo, plan.mtiles, plan.xcd};
  a.norm_w = static_cast<const uint16_t*>(norm_weight);
  a.norm_eps = eps;
  a.stagger = stagger_for(2 * I, K);
  hipStream_t s = as_stream(stream);
  if (norm) {
    if (dtype == RG_DTYPE_BF16) launch_gemm_silu_mul<bf16_t, true>(a, plan.nb, plan.mb, s);
    else launch_gemm_silu_mul<f16_t, true>(a, plan.nb, plan.mb, s);
  } else {
    if (dtype == RG_DTYPE_BF16) launch_gemm_silu_mul<bf16_t>(a, plan.nb, plan.mb, s);
    else launch_gemm_silu_mul<f16_t>(a, plan.nb, plan.mb, s);
  }
  return check_launch(op);
}

int qkv_rope_entry(const char* op, const void* x, const void* norm_weight, float eps, const void* weight_qkv,
                   void* q_out, void* k_cache, void* v_cache, const float* cos_sin, const int32_t* positions,
                   const int32_t* slot_mapping, int32_t M, int32_t num_heads, int32_t num_kv_heads, int32_t D,
                   int32_t block_size, int32_t K, int64_t ldx, int64_t ldw, int64_t ldq, int64_t kv_block_stride,
                   int32_t dtype, void* stream) {
  if (num_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 || num_heads % num_kv_heads != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: need positive heads (H a multiple of H_kv) and block_size", op);
  }
  if (D != 32 && D != 64) {
    return fail(RG_ERR_NOT_SUPPORTED, "%s: head_dim 32 or 64 (one head per column tile), got %d", op, D);
  }
  const int32_t N = (num_heads + 2 * num_kv_heads) * D;
  bool empty = false;
  if (int st = check_linear(op, x, weight_qkv, q_out, M, N, K, num_heads * D, ldx, ldw, ldq, dtype, empty)) {
    return st;
  }
  if (empty) return ok();
  if (!k_cache || !v_cache || !cos_sin || !positions || !slot_mapping) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  }
  const int64_t kv_stride = kv_block_stride ? kv_block_stride : (int64_t)num_kv_heads * block_size * D;
  if (kv_stride < (int64_t)num_kv_heads * block_size * D || !aligned16(k_cache) || !aligned16(v_cache) ||
      kv_stride % 8 != 0 || (reinterpret_cast<uintptr_t>(cos_sin) & 15u) != 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: cache block stride shorter than a block, or caches / cos_sin not "
                "16-byte aligned", op);
  }
  const int nb = D / 16;
  const bool norm = norm_weight != nullptr;
  const GemmPlan plan = gemm_plan(M, N, K, device_cu_count(), true, nb, norm);
  GemmArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(weight_qkv), static_cast<uint16_t*>(q_out),
             nullptr, M, N, K, ldx, ldw, ldq, plan.mtiles, plan.xcd,
             cos_sin, positions, slot_mapping, static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
             kv_stride, num_heads, num_kv_heads, block_size, static_cast<const uint16_t*>(norm_weight), eps,
             stagger_for(N, K)};
  hipStream_t s = as_stream(stream);
  if (norm) {
    if (dtype == RG_DTYPE_BF16) launch_gemm_rope<bf16_t, true>(a, nb, plan.mb, s);
    else launch_gemm_rope<f16_t, true>(a, nb, plan.mb, s);
  } else {
    if (dtype == RG_DTYPE_BF16) launch_gemm_rope<bf16_t>(a, nb, plan.mb, s);
    else launch_gemm_rope<f16_t>(a, nb, plan.mb, s);
  }
  return check_launch(op);
}
}  // namespace
}  // namespace rg

extern "C" int rg_linear(const void* x, const void* weight, void* out, int32_t num_rows, int32_t out_features,
                         int32_t in_features, int64_t x_row_stride, int64_t weight_row_stride,
                         int64_t out_row_stride, void* workspace, size_t workspace_bytes, int32_t dtype,
                         void* stream) {
  return linear_entry<kEpiPlain>("linear", x, weight, out, num_rows, out_features, in_features, x_row_stride,
                                 weight_row_stride, out_row_stride, workspace, workspace_bytes, dtype, stream);
}

extern "C" int rg_linear_residual(const void* x, const void* weight, void* residual, int32_t num_rows,
                                  int32_t out_features, int32_t in_features, int64_t x_row_stride,
                                  int64_t weight_row_stride, int64_t residual_row_stride, void* workspace,
                                  size_t workspace_bytes, int32_t dtype, void* stream) {
  return linear_entry<kEpiResidual>("linear_residual", x, weight, residual, num_rows, out_features, in_features,
                                    x_row_stride, weight_row_stride, residual_row_stride, workspace, workspace_bytes,
                                    dtype, stream);
}

extern "C" int rg_linear_silu_mul(const void* x, const void* weight_gate_up, void* out, int32_t num_rows,
                                  int32_t intermediate_size, int32_t in_features, int64_t x_row_stride,
                                  int64_t weight_row_stride, int64_t out_row_stride, int32_t dtype, void* stream) {
  return silu_mul_entry("linear_silu_mul", x, nullptr, 0.f, weight_gate_up, out, num_rows, intermediate_size,
                        in_features, x_row_stride, weight_row_stride, out_row_stride, dtype, stream);
}

extern "C" int rg_rms_norm_linear_silu_mul(const void* x, const void* norm_weight, float eps,
                                           const void* weight_gate_up, void* out, int32_t num_rows,
                                           int32_t intermediate_size, int32_t in_features, int64_t x_row_stride,
                                           int64_t weight_row_stride, int64_t out_row_stride, int32_t dtype,
                                           void* stream) {
  const char* op = "rms_norm_linear_silu_mul";
  if (num_rows > 0 && intermediate_size > 0) {
    if (int st = check_norm(op, norm_weight, in_features, eps)) return st;
  }
  return silu_mul_entry(op, x, norm_weight, eps, weight_gate_up, out, num_rows, intermediate_size, in_features,
                        x_row_stride, weight_row_stride, out_row_stride, dtype, stream);
}

extern "C" int rg_linear_qkv_rope_reshape_and_cache(const void* x, const void* weight_qkv, void* q_out,
                                                    void* k_cache, void* v_cache, const float* cos_sin,
                                                    const int32_t* positions, const int32_t* slot_mapping,
                                                    int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                                                    int32_t head_dim, int32_t block_size, int32_t in_features,
                                                    int64_t x_row_stride, int64_t weight_row_stride,
                                                    int64_t q_out_token_stride, int64_t kv_block_stride,
                                                    int32_t dtype, void* stream) {
  return qkv_rope_entry("linear_qkv_rope_reshape_and_cache", x, nullptr, 0.f, weight_qkv, q_out, k_cache, v_cache,
                        cos_sin, positions, slot_mapping, num_tokens, num_heads, num_kv_heads, head_dim, block_size,
                        in_features, x_row_stride, weight_row_stride, q_out_token_stride, kv_block_stride, dtype,
                        stream);
}

extern "C" int rg_rms_norm_linear_qkv_rope_reshape_and_cache(
    const void* x, const void* norm_weight, float eps, const void* weight_qkv, void* q_out, void* k_cache,
    void* v_cache, const float* cos_sin, const int32_t* positions, const int32_t* slot_mapping, int32_t num_tokens,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t in_features,
    int64_t x_row_stride, int64_t weight_row_stride, int64_t q_out_token_stride, int64_t kv_block_stride,
    int32_t dtype, void* stream) {
  const char* op = "rms_norm_linear_qkv_rope_reshape_and_cache";
  if (num_tokens > 0) {
    if (int st = check_norm(op, norm_weight, in_features, eps)) return st;
  }
  return qkv_rope_entry(op, x, norm_weight, eps, weight_qkv, q_out, k_cache, v_cache, cos_sin, positions,
                        slot_mapping, num_tokens, num_heads, num_kv_heads, head_dim, block_size, in_features,
                        x_row_stride, weight_row_stride, q_out_token_stride, kv_block_stride, dtype, stream);
}
