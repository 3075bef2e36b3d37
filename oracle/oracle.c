/*
 * oracle.c — CPU restatement of Railgun's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the GPU kernels are
 * compared against; only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load it.  The product (railgun_amd/) never calls it.
 *
 * Every function restates one piece of the reference's arithmetic or index
 * contract (file:line into the Railgun repository).  Element types: 0 = fp32,
 * 1 = bf16, 2 = fp16, always stored as raw bits and upcast to fp32 on load;
 * attention outputs are fp32.  Built with -ffp-contract=off so that products
 * and sums are rounded separately, as in the reference's C expressions.
 *
 * Pinning (what checks each function independently of this file) is listed
 * in the header of oracle/oracle.py and in tests/test_oracle.py.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_F32 0
#define OR_BF16 1
#define OR_F16 2
/* head_dim bound of the gathered prefill rows (larger ones take prefill_row) */
#define OR_MAX_GATHER_D 1024

/* ------------------------------------------------------------ elements ---- */

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

float or_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 */
    float v = (float)man * 5.9604644775390625e-08f;
    return (sign ? -v : v);
  }
  if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t or_f32_to_f16(float f) {
  const uint32_t u = f32_to_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t absu = u & 0x7fffffffu;
  if (absu > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);     /* NaN */
  if (absu >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);    /* overflow to inf (>= 65520) */
  if (absu < 0x38800000u) {
    /* subnormal half (or zero): round absu-as-float * 2^24 to an integer, RNE */
    const float a = bits_to_f32(absu);
    const float scaled = a * 16777216.0f; /* exact: power of two */
    float r = nearbyintf(scaled);          /* default rounding mode: nearest-even */
    return (uint16_t)(sign | (uint16_t)r);
  }
  uint32_t e = ((absu >> 23) - 112u) << 10;
  uint32_t m = (absu >> 13) & 0x3ffu;
  const uint32_t rest = absu & 0x1fffu;
  uint32_t out = e | m;
  if (rest > 0x1000u || (rest == 0x1000u && (m & 1u))) out += 1u;
  return (uint16_t)(sign | out);
}

static inline float ld(const void* p, int64_t i, int dt) {
  switch (dt) {
    case OR_BF16: return or_bf16_to_f32(((const uint16_t*)p)[i]);
    case OR_F16: return or_f16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

static inline void st(void* p, int64_t i, int dt, float v) {
  switch (dt) {
    case OR_BF16: ((uint16_t*)p)[i] = or_f32_to_bf16(v); break;
    case OR_F16: ((uint16_t*)p)[i] = or_f32_to_f16(v); break;
    default: ((float*)p)[i] = v; break;
  }
}

static inline int esize(int dt) { return dt == OR_F32 ? 4 : 2; }

/* Element offset of (block, kv-head, in-block offset) in a paged cache:
 * ((blk*H_kv + h)*bs + off)*D for the dense layout
 * (crates/vllm-cuda/src/kernels/paged_attention.cu:130-134), generalised to
 * an explicit block stride (0 = dense). */
static inline int64_t cache_row(int64_t blk, int h, int off, int Hkv, int bs, int D,
                                int64_t stride) {
  const int64_t s = stride ? stride : (int64_t)Hkv * bs * D;
  return blk * s + ((int64_t)h * bs + off) * D;
}

/* ------------------------------------------------------ reshape_and_cache -- */

/* crates/vllm-cuda/src/kernels/paged_attention.cu:121-137: for every token t
 * with slot >= 0, blk = slot / bs, off = slot % bs, copy the H_kv rows of k and
 * v (bit copies).  With `meta` != NULL also the identity IsoQuant metadata at
 * off == 0 (paged_attention.cu:168-173, isoquant_utils.cuh:54-58). */
void or_reshape_and_cache(const void* k, const void* v, void* kc, void* vc, const int32_t* slot,
                          float* meta, int T, int Hkv, int D, int bs, int dt, int64_t stride) {
  const int es = esize(dt);
  for (int t = 0; t < T; ++t) {
    const int32_t sl = slot[t];
    if (sl < 0) continue;
    const int64_t blk = sl / bs;
    const int off = sl % bs;
    for (int h = 0; h < Hkv; ++h) {
      const int64_t src = ((int64_t)t * Hkv + h) * D;
      const int64_t dst = cache_row(blk, h, off, Hkv, bs, D, stride);
      memcpy((char*)kc + dst * es, (const char*)k + src * es, (size_t)D * es);
      memcpy((char*)vc + dst * es, (const char*)v + src * es, (size_t)D * es);
    }
    if (meta && off == 0) {
      const int groups = Hkv * (D / 4);
      float* m = meta + blk * (int64_t)groups * 8;
      for (int g = 0; g < groups * 8; ++g) m[g] = ((g & 3) == 3) ? 1.f : 0.f;
    }
  }
}

/* ------------------------------------------------------------------ RoPE --- */

/* crates/vllm-cuda/src/kernels/rope.cu:18-41: for each pair (i, i+D/2),
 *   lo' = lo*c - hi*s,  hi' = hi*c + lo*s,
 *   c = cos_sin[pos*D + i], s = cos_sin[pos*D + D/2 + i],
 * every product rounded to fp32 before the add (-ffp-contract=off). */
static void rope_row(const void* src, int64_t src_off, void* dst, int64_t dst_off, const float* cs,
                     int D, int dt) {
  const int half = D / 2;
  for (int i = 0; i < half; ++i) {
    const float lo = ld(src, src_off + i, dt);
    const float hi = ld(src, src_off + half + i, dt);
    const float c = cs[i];
    const float s = cs[half + i];
    const float a = lo * c;
    const float b = hi * s;
    const float e = hi * c;
    const float f = lo * s;
    st(dst, dst_off + i, dt, a - b);
    st(dst, dst_off + half + i, dt, e + f);
  }
}

void or_rope(void* x, const float* cos_sin, const int32_t* pos, int T, int H, int D, int dt) {
  for (int t = 0; t < T; ++t) {
    const float* cs = cos_sin + (int64_t)pos[t] * D;
    for (int h = 0; h < H; ++h) {
      const int64_t off = ((int64_t)t * H + h) * D;
      rope_row(x, off, x, off, cs, D, dt);
    }
  }
}

/* RoPE on q in place, then RoPE on k and the scatter of rotated k and of v
 * (the order rope -> reshape_and_cache of attention.rs:119-125 once RoPE is
 * applied); k itself is not modified. */
void or_rope_reshape_and_cache(void* q, const void* k, const void* v, void* kc, void* vc,
                               const float* cos_sin, const int32_t* pos, const int32_t* slot,
                               int T, int H, int Hkv, int D, int bs, int dt, int64_t stride) {
  or_rope(q, cos_sin, pos, T, H, D, dt);
  const int es = esize(dt);
  for (int t = 0; t < T; ++t) {
    const int32_t sl = slot[t];
    if (sl < 0) continue;
    const int64_t blk = sl / bs;
    const int off = sl % bs;
    const float* cs = cos_sin + (int64_t)pos[t] * D;
    for (int h = 0; h < Hkv; ++h) {
      const int64_t src = ((int64_t)t * Hkv + h) * D;
      const int64_t dst = cache_row(blk, h, off, Hkv, bs, D, stride);
      rope_row(k, src, kc, dst, cs, D, dt);
      memcpy((char*)vc + dst * es, (const char*)v + src * es, (size_t)D * es);
    }
  }
}

/* ------------------------------------------------------------- decode ------ */

typedef struct {
  const void* q;
  const void* kc;
  const void* vc;
  const int32_t* bt;
  const int32_t* ctx;
  float scale;
  int B, H, Hkv, D, bs, MB, dt;
  int64_t stride;
} dec_args;

static inline int64_t token_row(const dec_args* a, int s, int kvh, int t) {
  const int64_t blk = a->bt[(int64_t)s * a->MB + t / a->bs];
  return cache_row(blk, kvh, t % a->bs, a->Hkv, a->bs, a->D, a->stride);
}

static float dot_qk(const dec_args* a, const float* q, int64_t row) {
  float acc = 0.f;
  for (int d = 0; d < a->D; ++d) acc += q[d] * ld(a->kc, row + d, a->dt);
  return acc;
}

static void load_q(const dec_args* a, int s, int h, float* q) {
  for (int d = 0; d < a->D; ++d) q[d] = ld(a->q, ((int64_t)s * a->H + h) * a->D + d, a->dt);
}

/* crates/vllm-cuda/src/kernels/paged_attention.cu:33-107 (two-pass v1):
 * kvh = h / (H/H_kv) (:40); pass 1 keeps a running max l_max (from -1e20) and
 * a running sum l_sum (:54-78); pass 2 recomputes every score and accumulates
 * exp(score - l_max) * V (:84-105); out = res / l_sum (:107).  ctx == 0 gives
 * zeros here, where the reference divides 0/0 (a NaN) — the single-pass and
 * split-K kernels, which production uses, give zeros. */
void or_paged_attention_v1(const void* q, const void* kc, const void* vc, const int32_t* bt,
                           const int32_t* ctx, float* out, float scale, int B, int H, int Hkv,
                           int D, int bs, int MB, int dt, int64_t stride) {
  dec_args a = {q, kc, vc, bt, ctx, scale, B, H, Hkv, D, bs, MB, dt, stride};
  float* qv = (float*)malloc(sizeof(float) * D);
  for (int s = 0; s < B; ++s) {
    for (int h = 0; h < H; ++h) {
      const int kvh = h / (H / Hkv);
      float* o = out + ((int64_t)s * H + h) * D;
      const int n = ctx[s];
      if (n <= 0) {
        memset(o, 0, sizeof(float) * D);
        continue;
      }
      load_q(&a, s, h, qv);
      float l_max = -1e20f, l_sum = 0.f;
      for (int t = 0; t < n; ++t) {
        const float sc = dot_qk(&a, qv, token_row(&a, s, kvh, t)) * scale;
        const float old = l_max;
        l_max = fmaxf(l_max, sc);
        l_sum = l_sum * expf(old - l_max) + expf(sc - l_max);
      }
      for (int d = 0; d < D; ++d) {
        float res = 0.f;
        for (int t = 0; t < n; ++t) {
          const int64_t row = token_row(&a, s, kvh, t);
          const float sc = dot_qk(&a, qv, row) * scale;
          res += expf(sc - l_max) * ld(vc, row + d, dt);
        }
        o[d] = res / l_sum;
      }
    }
  }
  free(qv);
}

/* Online-softmax pass over tokens [t0, t1) of (s, h):
 * crates/vllm-cuda/src/kernels/paged_attention_v1_plus.cu:52-92 (and the same
 * loop in paged_attention_v2_partition.cu:162-199): m from -inf, per token
 *   m' = max(m, x); s = s*exp(m-m') + exp(x-m'); o = o*exp(m-m') + exp(x-m')*v. */
static void online_pass(const dec_args* a, int s, int h, int t0, int t1, const float* qv,
                        float* m_out, float* s_out, float* o) {
  const int kvh = h / (a->H / a->Hkv);
  float m = -INFINITY, sum = 0.f;
  for (int d = 0; d < a->D; ++d) o[d] = 0.f;
  for (int t = t0; t < t1; ++t) {
    const int64_t row = token_row(a, s, kvh, t);
    const float x = dot_qk(a, qv, row) * a->scale;
    const float m_old = m;
    m = fmaxf(m, x);
    const float e_m = expf(m_old - m);
    const float e_x = expf(x - m);
    sum = sum * e_m + e_x;
    for (int d = 0; d < a->D; ++d) o[d] = o[d] * e_m + e_x * ld(a->vc, row + d, a->dt);
  }
  *m_out = m;
  *s_out = sum;
}

/* crates/vllm-cuda/src/kernels/paged_attention_v1_plus.cu:37-105 (single pass,
 * identity rotation): ctx == 0 leaves the zero-filled output (:38), the
 * division is skipped when the sum is 0 (:95-100). */
void or_paged_attention_v1_plus(const void* q, const void* kc, const void* vc, const int32_t* bt,
                                const int32_t* ctx, float* out, float scale, int B, int H,
                                int Hkv, int D, int bs, int MB, int dt, int64_t stride) {
  dec_args a = {q, kc, vc, bt, ctx, scale, B, H, Hkv, D, bs, MB, dt, stride};
  float* qv = (float*)malloc(sizeof(float) * D);
  for (int s = 0; s < B; ++s) {
    for (int h = 0; h < H; ++h) {
      float* o = out + ((int64_t)s * H + h) * D;
      if (ctx[s] <= 0) {
        memset(o, 0, sizeof(float) * D);
        continue;
      }
      load_q(&a, s, h, qv);
      float m, sum;
      online_pass(&a, s, h, 0, ctx[s], qv, &m, &sum, o);
      if (sum != 0.f)
        for (int d = 0; d < D; ++d) o[d] /= sum;
    }
  }
  free(qv);
}

/* crates/vllm-cuda/src/kernels/paged_attention_v2_partition.cu:37-106 with the
 * partition size P as a parameter (the reference fixes 256,
 * paged_attention_utils.cuh:10): partition p covers [p*P, min((p+1)*P, ctx));
 * partitions past the context are not written (:146). */
void or_paged_attention_v2_partition(const void* q, const void* kc, const void* vc,
                                     const int32_t* bt, const int32_t* ctx, float* tmp_out,
                                     float* exp_sums, float* max_logits, float scale, int B,
                                     int H, int Hkv, int D, int bs, int MB, int NP, int P, int dt,
                                     int64_t stride) {
  dec_args a = {q, kc, vc, bt, ctx, scale, B, H, Hkv, D, bs, MB, dt, stride};
  float* qv = (float*)malloc(sizeof(float) * D);
  for (int s = 0; s < B; ++s) {
    for (int h = 0; h < H; ++h) {
      load_q(&a, s, h, qv);
      for (int p = 0; p < NP; ++p) {
        const int t0 = p * P;
        if (t0 >= ctx[s]) continue;
        const int t1 = t0 + P < ctx[s] ? t0 + P : ctx[s];
        const int64_t sh = ((int64_t)s * H + h) * NP + p;
        online_pass(&a, s, h, t0, t1, qv, &max_logits[sh], &exp_sums[sh], tmp_out + sh * D);
      }
    }
  }
  free(qv);
}

/* crates/vllm-cuda/src/kernels/paged_attention_v2_reduce.cu:27-95 without the
 * 512-partition cap: NP_s = ceil(ctx/P); M = max m_p; r_p = exp(m_p - M);
 * S = sum r_p l_p; out = sum r_p tmp_p / S (division skipped when S == 0);
 * ctx == 0 writes zeros (:30-36). */
void or_paged_attention_v2_reduce(float* out, const float* exp_sums, const float* max_logits,
                                  const float* tmp_out, const int32_t* ctx, int B, int H, int D,
                                  int NP, int P) {
  for (int s = 0; s < B; ++s) {
    const int nps = ctx[s] > 0 ? (ctx[s] + P - 1) / P : 0;
    for (int h = 0; h < H; ++h) {
      float* o = out + ((int64_t)s * H + h) * D;
      for (int d = 0; d < D; ++d) o[d] = 0.f;
      if (nps == 0) continue;
      const int64_t sh = ((int64_t)s * H + h) * NP;
      float M = -INFINITY;
      for (int p = 0; p < nps; ++p) M = fmaxf(M, max_logits[sh + p]);
      float S = 0.f;
      for (int p = 0; p < nps; ++p) S += expf(max_logits[sh + p] - M) * exp_sums[sh + p];
      for (int p = 0; p < nps; ++p) {
        const float r = expf(max_logits[sh + p] - M);
        for (int d = 0; d < D; ++d) o[d] += r * tmp_out[(sh + p) * D + d];
      }
      if (S != 0.f)
        for (int d = 0; d < D; ++d) o[d] /= S;
    }
  }
}

/* ------------------------------------------------------------- prefill ----- */

/* Textbook causal attention for a packed stream (the reference has no prefill
 * kernel; crates/vllm-models/src/llama/attention.rs:128-132 routes prefill
 * through the decode op).  Row j of sequence s (rows cu[s]..cu[s+1]) sits at
 * position ctx[s] - L_s + j and attends to cache positions 0..pos with
 * softmax(scale * q.K) V, computed in double.  GQA kvh = h / (H/H_kv).
 *
 * prefill_row computes every head of one packed row; sc holds pos + 1 doubles
 * and acc D doubles. */
static void prefill_row(const dec_args* a, const int32_t* cu, float* out, int s, int row,
                        double* sc, double* acc) {
  const int L = cu[s + 1] - cu[s];
  const int pos = a->ctx[s] - L + (row - cu[s]);
  const int H = a->H, D = a->D;
  for (int h = 0; h < H; ++h) {
    float* o = out + ((int64_t)row * H + h) * D;
    if (pos < 0) {
      memset(o, 0, sizeof(float) * D);
      continue;
    }
    const int kvh = h / (H / a->Hkv);
    double mx = -INFINITY;
    for (int t = 0; t <= pos; ++t) {
      const int64_t r = token_row(a, s, kvh, t);
      double dot = 0.0;
      for (int d = 0; d < D; ++d)
        dot += (double)ld(a->q, ((int64_t)row * H + h) * D + d, a->dt) * (double)ld(a->kc, r + d, a->dt);
      sc[t] = dot * (double)a->scale;
      if (sc[t] > mx) mx = sc[t];
    }
    double sum = 0.0;
    for (int d = 0; d < D; ++d) acc[d] = 0.0;
    for (int t = 0; t <= pos; ++t) {
      const double e = exp(sc[t] - mx);
      sum += e;
      const int64_t r = token_row(a, s, kvh, t);
      for (int d = 0; d < D; ++d) acc[d] += e * (double)ld(a->vc, r + d, a->dt);
    }
    for (int d = 0; d < D; ++d) o[d] = (float)(acc[d] / sum);
  }
}

static int max_ctx_of(const int32_t* ctx, int S) {
  int m = 1;
  for (int s = 0; s < S; ++s)
    if (ctx[s] > m) m = ctx[s];
  return m;
}

void or_prefill_packed(const void* q, const void* kc, const void* vc, const int32_t* bt,
                       const int32_t* ctx, const int32_t* cu, float* out, float scale, int S,
                       int H, int Hkv, int D, int bs, int MB, int dt, int64_t stride) {
  dec_args a = {q, kc, vc, bt, ctx, scale, S, H, Hkv, D, bs, MB, dt, stride};
  double* sc = (double*)malloc(sizeof(double) * (size_t)max_ctx_of(ctx, S));
  double* acc = (double*)malloc(sizeof(double) * D);
  for (int s = 0; s < S; ++s)
    for (int row = cu[s]; row < cu[s + 1]; ++row) prefill_row(&a, cu, out, s, row, sc, acc);
  free(sc);
  free(acc);
}

/* The same rows as or_prefill_packed, for a list of packed row indices only
 * (rows[i] in [0, cu[S])), spread over `nthreads` POSIX threads: every listed
 * row of `out` is written exactly as or_prefill_packed writes it, the others
 * are left untouched.  For long streams where every row would take minutes.
 *
 * Speed only: the K and V rows of every (sequence, kv-head) that a listed row
 * needs are first gathered once into contiguous fp32 arrays [ctx, D] (the
 * values ld() returns), so the per-row loops read plain floats.  The products,
 * sums and their order are those of prefill_row, so the results are the same
 * bits (tests/test_oracle.py checks this). */
typedef struct {
  const dec_args* a;
  const int32_t* cu;
  const int32_t* rows;
  float* out;
  float** kg; /* [s * Hkv + kvh] -> gathered K rows [ctx_s, D] (NULL if unused) */
  float** vg;
  int nrows;
  int next;
  pthread_mutex_t mu;
} prefill_job;

static void prefill_row_gathered(const prefill_job* job, int s, int row, double* sc, double* acc) {
  const dec_args* a = job->a;
  const int L = job->cu[s + 1] - job->cu[s];
  const int pos = a->ctx[s] - L + (row - job->cu[s]);
  const int H = a->H, D = a->D;
  for (int h = 0; h < H; ++h) {
    float* o = job->out + ((int64_t)row * H + h) * D;
    if (pos < 0) {
      memset(o, 0, sizeof(float) * D);
      continue;
    }
    const int kvh = h / (H / a->Hkv);
    const float* K = job->kg[(int64_t)s * a->Hkv + kvh];
    const float* V = job->vg[(int64_t)s * a->Hkv + kvh];
    double qd[OR_MAX_GATHER_D];
    for (int d = 0; d < D; ++d) qd[d] = (double)ld(a->q, ((int64_t)row * H + h) * D + d, a->dt);
    double mx = -INFINITY;
    for (int t = 0; t <= pos; ++t) {
      const float* kr = K + (int64_t)t * D;
      double dot = 0.0;
      for (int d = 0; d < D; ++d) dot += qd[d] * (double)kr[d];
      sc[t] = dot * (double)a->scale;
      if (sc[t] > mx) mx = sc[t];
    }
    double sum = 0.0;
    for (int d = 0; d < D; ++d) acc[d] = 0.0;
    for (int t = 0; t <= pos; ++t) {
      const double e = exp(sc[t] - mx);
      sum += e;
      const float* vr = V + (int64_t)t * D;
      for (int d = 0; d < D; ++d) acc[d] += e * (double)vr[d];
    }
    for (int d = 0; d < D; ++d) o[d] = (float)(acc[d] / sum);
  }
}

static void* prefill_worker(void* arg) {
  prefill_job* job = (prefill_job*)arg;
  const dec_args* a = job->a;
  double* sc = (double*)malloc(sizeof(double) * (size_t)max_ctx_of(a->ctx, a->B));
  double* acc = (double*)malloc(sizeof(double) * a->D);
  for (;;) {
    pthread_mutex_lock(&job->mu);
    const int i = job->next++;
    pthread_mutex_unlock(&job->mu);
    if (i >= job->nrows) break;
    const int row = job->rows[i];
    int s = 0;
    while (s + 1 < a->B && job->cu[s + 1] <= row) ++s;
    if (a->D <= OR_MAX_GATHER_D) prefill_row_gathered(job, s, row, sc, acc);
    else prefill_row(a, job->cu, job->out, s, row, sc, acc);
  }
  free(sc);
  free(acc);
  return NULL;
}

void or_prefill_packed_rows(const void* q, const void* kc, const void* vc, const int32_t* bt,
                            const int32_t* ctx, const int32_t* cu, const int32_t* rows, int nrows,
                            float* out, float scale, int S, int H, int Hkv, int D, int bs, int MB,
                            int dt, int64_t stride, int nthreads) {
  dec_args a = {q, kc, vc, bt, ctx, scale, S, H, Hkv, D, bs, MB, dt, stride};
  prefill_job job;
  job.a = &a;
  job.cu = cu;
  job.rows = rows;
  job.out = out;
  job.nrows = nrows;
  job.next = 0;
  job.kg = (float**)calloc((size_t)S * Hkv, sizeof(float*));
  job.vg = (float**)calloc((size_t)S * Hkv, sizeof(float*));
  /* Gather the (sequence, kv-head) rows the listed rows read: positions 0 .. ctx - 1. */
  if (D <= OR_MAX_GATHER_D) {
    for (int i = 0; i < nrows; ++i) {
      int s = 0;
      while (s + 1 < S && cu[s + 1] <= rows[i]) ++s;
      if (job.kg[(int64_t)s * Hkv] || ctx[s] <= 0) continue;
      for (int h = 0; h < Hkv; ++h) {
        float* K = (float*)malloc(sizeof(float) * (size_t)ctx[s] * D);
        float* V = (float*)malloc(sizeof(float) * (size_t)ctx[s] * D);
        for (int t = 0; t < ctx[s]; ++t) {
          const int64_t r = token_row(&a, s, h, t);
          for (int d = 0; d < D; ++d) {
            K[(int64_t)t * D + d] = ld(kc, r + d, dt);
            V[(int64_t)t * D + d] = ld(vc, r + d, dt);
          }
        }
        job.kg[(int64_t)s * Hkv + h] = K;
        job.vg[(int64_t)s * Hkv + h] = V;
      }
    }
  }
  pthread_mutex_init(&job.mu, NULL);
  if (nthreads < 1) nthreads = 1;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * nthreads);
  for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, prefill_worker, &job);
  for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
  free(th);
  pthread_mutex_destroy(&job.mu);
  for (int64_t i = 0; i < (int64_t)S * Hkv; ++i) {
    free(job.kg[i]);
    free(job.vg[i]);
  }
  free(job.kg);
  free(job.vg);
}

/* ------------------------------------------- reference CPU attention path --- */

/* The reference's CPU counterpart of the decode op, "candle-core CPU attention
 * over the gathered blocks" (the rank-3 path of attention.rs:144-154 fed with
 * gathered cache rows): per (s, kv-head) gather the ctx rows of K and V into
 * contiguous fp32 [ctx, D] (candle's to_dtype(F32) of the gathered tensor); per
 * q-head scores = q.K^T * scale (attention.rs:150), softmax over the last dim
 * (max-subtract, exp, sum, divide; attention.rs:151), out = probs.V
 * (attention.rs:152).  Work items (s, kv-head) are spread over `nthreads` POSIX
 * threads.
 *
 * The two products are written the way a blocked CPU gemm (candle's `gemm`
 * crate) computes them: q.K^T with eight-lane partial sums over d, all G q-heads
 * of the kv-head from one load of each K row, and probs.V as rank-1 updates over
 * t.  The dot products are therefore summed in a different order than a
 * sequential loop (a float32 rounding difference, covered by the tolerance of
 * every comparison).  The hot loops are compiled for AVX2 and for generic
 * x86-64, picked at load time. */
typedef struct {
  const dec_args* a;
  float* out;
  int next;
  int n_items;
  pthread_mutex_t mu;
} cpu_job;

#if defined(__x86_64__) && defined(__GNUC__) && !defined(__clang__)
#define OR_CLONES __attribute__((target_clones("avx2", "default")))
#else
#define OR_CLONES
#endif

typedef float v8f __attribute__((vector_size(32)));

static inline v8f ld8(const float* p) {
  v8f v;
  memcpy(&v, p, sizeof(v));
  return v;
}

/* sc[j][t] = (q_j . K[t]) * scale for the g q-heads q [g, D] and rows K [n, D]
 * (D a multiple of 8). */
OR_CLONES static void scores_group(const float* restrict q, const float* restrict kg, float* restrict sc, int n,
                                   int D, int g, float scale) {
  for (int t = 0; t < n; ++t) {
    const float* restrict kr = kg + (int64_t)t * D;
    for (int j0 = 0; j0 < g; j0 += 4) {
      const int nj = g - j0 < 4 ? g - j0 : 4;
      v8f acc[4] = {{0}, {0}, {0}, {0}};
      for (int d = 0; d < D; d += 8) {
        const v8f k8 = ld8(kr + d);
        for (int j = 0; j < nj; ++j) acc[j] += ld8(q + (int64_t)(j0 + j) * D + d) * k8;
      }
      for (int j = 0; j < nj; ++j) {
        const v8f a = acc[j];
        const float sum = ((a[0] + a[4]) + (a[1] + a[5])) + ((a[2] + a[6]) + (a[3] + a[7]));
        sc[(int64_t)(j0 + j) * n + t] = sum * scale;
      }
    }
  }
}

/* o[j][d] = sum_t p[j][t] * V[t][d] for the g heads, accumulated in t order; 16-column
 * slices of four heads are held in registers over the whole t loop (D a multiple of 16). */
OR_CLONES static void probs_v_group(const float* restrict p, const float* restrict vg, float* restrict o, int n,
                                    int D, int g) {
  for (int d0 = 0; d0 < D; d0 += 16) {
    for (int j0 = 0; j0 < g; j0 += 4) {
      const int nj = g - j0 < 4 ? g - j0 : 4;
      v8f acc[4][2] = {{{0}, {0}}, {{0}, {0}}, {{0}, {0}}, {{0}, {0}}};
      for (int t = 0; t < n; ++t) {
        const float* restrict vr = vg + (int64_t)t * D + d0;
        const v8f v0 = ld8(vr), v1 = ld8(vr + 8);
        for (int j = 0; j < nj; ++j) {
          const float pt = p[(int64_t)(j0 + j) * n + t];
          acc[j][0] += pt * v0;
          acc[j][1] += pt * v1;
        }
      }
      for (int j = 0; j < nj; ++j) {
        memcpy(o + (int64_t)(j0 + j) * D + d0, &acc[j][0], sizeof(v8f));
        memcpy(o + (int64_t)(j0 + j) * D + d0 + 8, &acc[j][1], sizeof(v8f));
      }
    }
  }
}

/* The same for any D (a multiple of 4): rank-1 updates of o over t. */
static void probs_v_any(const float* restrict p, const float* restrict vg, float* restrict o, int n, int D, int g) {
  for (int i = 0; i < g * D; ++i) o[i] = 0.f;
  for (int t = 0; t < n; ++t)
    for (int j = 0; j < g; ++j) {
      const float pt = p[(int64_t)j * n + t];
      for (int d = 0; d < D; ++d) o[(int64_t)j * D + d] += pt * vg[(int64_t)t * D + d];
    }
}

/* One gathered row of K and of V as fp32. */
OR_CLONES static void gather_row(const void* kc, const void* vc, int64_t row, int D, int dt, float* restrict kr,
                                 float* restrict vr) {
  if (dt == OR_BF16) {
    const uint16_t* kp = (const uint16_t*)kc + row;
    const uint16_t* vp = (const uint16_t*)vc + row;
    for (int d = 0; d < D; ++d) {
      kr[d] = bits_to_f32((uint32_t)kp[d] << 16);
      vr[d] = bits_to_f32((uint32_t)vp[d] << 16);
    }
  } else {
    for (int d = 0; d < D; ++d) {
      kr[d] = ld(kc, row + d, dt);
      vr[d] = ld(vc, row + d, dt);
    }
  }
}

/* Scratch per thread: kg/vg [n, D], probs [g, n], qv and ov [g, D]. */
static void cpu_item(const dec_args* a, float* out, int item, float* kg, float* vg, float* probs,
                     float* qv, float* ov) {
  const int s = item / a->Hkv;
  const int kvh = item % a->Hkv;
  const int n = a->ctx[s] > 0 ? a->ctx[s] : 0;
  const int g = a->H / a->Hkv;
  const int D = a->D;
  float* o = out + ((int64_t)s * a->H + (int64_t)kvh * g) * D;  /* the group's g rows, contiguous */
  if (n == 0) {
    memset(o, 0, sizeof(float) * (size_t)g * D);
    return;
  }
  for (int t = 0; t < n; ++t)
    gather_row(a->kc, a->vc, token_row(a, s, kvh, t), D, a->dt, kg + (int64_t)t * D, vg + (int64_t)t * D);
  for (int j = 0; j < g; ++j) load_q(a, s, kvh * g + j, qv + (int64_t)j * D);
  if (D % 8 == 0) {
    scores_group(qv, kg, probs, n, D, g, a->scale);
  } else {
    for (int j = 0; j < g; ++j)
      for (int t = 0; t < n; ++t) {
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot += qv[(int64_t)j * D + d] * kg[(int64_t)t * D + d];
        probs[(int64_t)j * n + t] = dot * a->scale;
      }
  }
  for (int j = 0; j < g; ++j) {
    float* pj = probs + (int64_t)j * n;
    float mx = -INFINITY;
    for (int t = 0; t < n; ++t)
      if (pj[t] > mx) mx = pj[t];
    float sum = 0.f;
    for (int t = 0; t < n; ++t) {
      pj[t] = expf(pj[t] - mx);
      sum += pj[t];
    }
    for (int t = 0; t < n; ++t) pj[t] /= sum;
  }
  if (D % 16 == 0)
    probs_v_group(probs, vg, ov, n, D, g);
  else
    probs_v_any(probs, vg, ov, n, D, g);
  memcpy(o, ov, sizeof(float) * (size_t)g * D);
}

static void* cpu_worker(void* arg) {
  cpu_job* job = (cpu_job*)arg;
  const dec_args* a = job->a;
  int max_ctx = 0;
  for (int s = 0; s < a->B; ++s)
    if (a->ctx[s] > max_ctx) max_ctx = a->ctx[s];
  const size_t n = (size_t)(max_ctx > 0 ? max_ctx : 1);
  const size_t g = (size_t)(a->H / a->Hkv);
  float* kg = (float*)malloc(sizeof(float) * n * a->D);
  float* vg = (float*)malloc(sizeof(float) * n * a->D);
  float* probs = (float*)malloc(sizeof(float) * n * g);
  float* qv = (float*)malloc(sizeof(float) * g * a->D);
  float* ov = (float*)malloc(sizeof(float) * g * a->D);
  for (;;) {
    pthread_mutex_lock(&job->mu);
    const int item = job->next++;
    pthread_mutex_unlock(&job->mu);
    if (item >= job->n_items) break;
    cpu_item(a, job->out, item, kg, vg, probs, qv, ov);
  }
  free(kg);
  free(vg);
  free(probs);
  free(qv);
  free(ov);
  return NULL;
}

void or_cpu_attention_gathered(const void* q, const void* kc, const void* vc, const int32_t* bt,
                               const int32_t* ctx, float* out, float scale, int B, int H, int Hkv,
                               int D, int bs, int MB, int dt, int64_t stride, int nthreads) {
  dec_args a = {q, kc, vc, bt, ctx, scale, B, H, Hkv, D, bs, MB, dt, stride};
  cpu_job job;
  job.a = &a;
  job.out = out;
  job.next = 0;
  job.n_items = B * Hkv;
  pthread_mutex_init(&job.mu, NULL);
  if (nthreads < 1) nthreads = 1;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * nthreads);
  for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, cpu_worker, &job);
  for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
  free(th);
  pthread_mutex_destroy(&job.mu);
}
