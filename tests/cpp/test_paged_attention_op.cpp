// Tests of the C++ host mirror (include/railgun_hip.hpp) on the GPU: the op and the
// launchers called the way Railgun's Rust layer calls them (crates/vllm-cuda/src/kernels/
// paged_attn_op.rs:45-268, tests/test_paged_attention.rs:82-161), checked against host
// computations written here from the textbook definitions:
//   - reshape_and_cache (plain and IsoQuant): whole caches bit-exact against a host scatter,
//     slot -1 skipped, identity rotation metadata at block offset 0;
//   - execute(): the v1 branch (max_context_len <= 4096) and the v2 branch (longer), fp32
//     within 1e-4 and bf16 within 2e-2 abs + 1e-2 rel of double-precision attention, through
//     Railgun's fused [NB, 2, H_kv, bs, D] pool views;
//   - apply_rope against host rotate-half; prefill_packed against host causal attention;
//   - CoreError variants: NotSupported for head_dim 66, Tensor for a bad argument.
// Prints one line per check and exits non-zero on the first failure.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <vector>

#include "railgun_hip.hpp"

using railgun::CoreError;
using railgun::DeviceBuffer;
using railgun::DType;
using railgun::TensorView;

namespace {

int g_checks = 0;

void require(bool ok, const char* what) {
  ++g_checks;
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s\n", what);
    std::exit(1);
  }
  std::printf("ok   %s\n", what);
}

// splitmix64 -> uniform -> Box-Muller normal.
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
  float normal() {
    const double u1 = uniform(), u2 = uniform();
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
  int below(int n) { return (int)(next() % (uint64_t)n); }
};

uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
float from_bf16(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Shuffled block tables: sequence s takes the next ceil(ctx/bs) ids of a permutation of
// [0, nb); rows padded with 0.
std::vector<int32_t> block_tables(const std::vector<int32_t>& ctx, int bs, int nb, int mb, Rng& rng) {
  std::vector<int32_t> perm(nb);
  for (int i = 0; i < nb; ++i) perm[i] = i;
  for (int i = nb - 1; i > 0; --i) std::swap(perm[i], perm[rng.below(i + 1)]);
  std::vector<int32_t> bt(ctx.size() * mb, 0);
  int next = 0;
  for (size_t s = 0; s < ctx.size(); ++s)
    for (int b = 0; b < (ctx[s] + bs - 1) / bs; ++b) bt[s * mb + b] = perm[next++];
  return bt;
}

// Textbook decode attention in double over a pool laid out [NB, 2, H_kv, bs, D] (K at
// pair index 0, V at 1); `val` reads one stored element as float.
template <typename F>
std::vector<double> attention(const std::vector<float>& q, const F& val, const std::vector<int32_t>& bt,
                              const std::vector<int32_t>& ctx, int H, int hkv, int D, int bs, int mb,
                              double scale) {
  const int B = (int)ctx.size(), g = H / hkv;
  std::vector<double> out((size_t)B * H * D, 0.0);
  for (int s = 0; s < B; ++s) {
    const int n = ctx[s];
    if (n == 0) continue;
    for (int h = 0; h < H; ++h) {
      const int kvh = h / g;
      std::vector<double> sc(n);
      double m = -1e300;
      for (int t = 0; t < n; ++t) {
        const size_t row = (((size_t)bt[s * mb + t / bs] * 2 + 0) * hkv + kvh) * bs + t % bs;
        double acc = 0;
        for (int d = 0; d < D; ++d) acc += (double)q[((size_t)s * H + h) * D + d] * val(row * D + d);
        sc[t] = acc * scale;
        m = std::max(m, sc[t]);
      }
      double l = 0;
      for (int t = 0; t < n; ++t) l += (sc[t] = std::exp(sc[t] - m));
      for (int t = 0; t < n; ++t) {
        const size_t row = (((size_t)bt[s * mb + t / bs] * 2 + 1) * hkv + kvh) * bs + t % bs;
        for (int d = 0; d < D; ++d) out[((size_t)s * H + h) * D + d] += sc[t] / l * val(row * D + d);
      }
    }
  }
  return out;
}

double max_excess(const std::vector<double>& want, const std::vector<float>& got, double abs_tol,
                  double rel_tol) {
  double worst = 0;
  for (size_t i = 0; i < want.size(); ++i) {
    const double err = std::fabs(want[i] - (double)got[i]);
    const double tol = abs_tol + rel_tol * std::fabs(want[i]);
    if (!(err <= tol)) worst = std::max(worst, std::isnan(err) ? 1e30 : err - tol);
  }
  return worst;
}

// Pool views of Railgun's fused layout [NB, 2, H_kv, bs, D] (block.rs:70,89-95).
TensorView pool_view(void* base, DType dt, int nb, int hkv, int bs, int D, int which) {
  TensorView t = TensorView::contiguous(base, dt, {nb, hkv, bs, D});
  t.data = static_cast<char*>(base) + (size_t)which * hkv * bs * D * railgun::dtype_size(dt);
  t.strides[0] = 2LL * hkv * bs * D;
  return t;
}

void test_decode(const std::shared_ptr<railgun::PagedAttentionKernels>& kern, DType dt, int max_ctx, int seed) {
  const int H = 32, hkv = 8, D = 128, bs = 16, B = 6;
  Rng rng(seed);
  std::vector<int32_t> ctx(B);
  for (int s = 0; s < B; ++s) ctx[s] = 1 + rng.below(max_ctx);
  ctx[0] = max_ctx;   // the dispatch rule looks at the longest context
  ctx[B - 1] = 0;     // an empty sequence gives zeros
  int need = 0, mctx = 0;
  for (int c : ctx) need += (c + bs - 1) / bs, mctx = std::max(mctx, c);
  const int nb = need + 7, mb = (mctx + bs - 1) / bs + 2;
  const std::vector<int32_t> bt = block_tables(ctx, bs, nb, mb, rng);
  const size_t pool_elems = (size_t)nb * 2 * hkv * bs * D;
  std::vector<float> q((size_t)B * H * D), pool(pool_elems);
  for (auto& x : q) x = rng.normal();
  for (auto& x : pool) x = rng.normal();
  const double scale = 1.0 / std::sqrt((double)D);

  const size_t es = railgun::dtype_size(dt);
  DeviceBuffer<uint8_t> dq(q.size() * es), dpool(pool_elems * es);
  std::vector<double> want;
  if (dt == DType::F32) {
    dq.copy_from_host(std::vector<uint8_t>((uint8_t*)q.data(), (uint8_t*)q.data() + q.size() * 4));
    dpool.copy_from_host(std::vector<uint8_t>((uint8_t*)pool.data(), (uint8_t*)pool.data() + pool_elems * 4));
    want = attention(q, [&](size_t i) { return (double)pool[i]; }, bt, ctx, H, hkv, D, bs, mb, scale);
  } else {
    std::vector<uint16_t> qb(q.size()), pb(pool_elems);
    for (size_t i = 0; i < q.size(); ++i) qb[i] = to_bf16(q[i]), q[i] = from_bf16(qb[i]);
    for (size_t i = 0; i < pool_elems; ++i) pb[i] = to_bf16(pool[i]);
    dq.copy_from_host(std::vector<uint8_t>((uint8_t*)qb.data(), (uint8_t*)qb.data() + qb.size() * 2));
    dpool.copy_from_host(std::vector<uint8_t>((uint8_t*)pb.data(), (uint8_t*)pb.data() + pb.size() * 2));
    want = attention(q, [&](size_t i) { return (double)from_bf16(pb[i]); }, bt, ctx, H, hkv, D, bs, mb, scale);
  }
  auto dbt = DeviceBuffer<int32_t>::from_host(bt);
  auto dctx = DeviceBuffer<int32_t>::from_host(ctx);

  railgun::PagedAttentionOp op((float)scale, H, hkv, D, bs, kern);
  DeviceBuffer<uint8_t> out = op.execute(TensorView::contiguous(dq.data(), dt, {B, H, D}),
                                         pool_view(dpool.data(), dt, nb, hkv, bs, D, 0),
                                         pool_view(dpool.data(), dt, nb, hkv, bs, D, 1),
                                         TensorView::contiguous(dbt.data(), DType::F32, {B, mb}),
                                         TensorView::contiguous(dctx.data(), DType::F32, {B}), nullptr, mctx);
  const std::vector<uint8_t> raw = out.to_host();
  std::vector<float> got(want.size());
  if (dt == DType::F32) {
    std::memcpy(got.data(), raw.data(), got.size() * 4);
  } else {
    for (size_t i = 0; i < got.size(); ++i) got[i] = from_bf16((uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8)));
  }
  const double excess = dt == DType::F32 ? max_excess(want, got, 1e-4, 1e-4) : max_excess(want, got, 2e-2, 1e-2);
  char what[160];
  std::snprintf(what, sizeof what, "execute %s, %s branch (max_context_len %d, fused pool views)",
                dt == DType::F32 ? "fp32" : "bf16", mctx <= 4096 ? "v1" : "v2", mctx);
  require(excess == 0.0, what);
  bool zero_row = true;
  for (int i = 0; i < H * D; ++i) zero_row &= got[(size_t)(B - 1) * H * D + i] == 0.f;
  require(zero_row, "execute: context length 0 gives zeros");
}

void test_cache_and_rope(const std::shared_ptr<railgun::PagedAttentionKernels>& kern) {
  const int hkv = 8, D = 64, bs = 16, nb = 32, T = 9, H = 32;
  Rng rng(1001);
  std::vector<float> k((size_t)T * hkv * D), v(k.size()), kc((size_t)nb * hkv * bs * D), vc(kc.size());
  for (auto& x : k) x = rng.normal();
  for (auto& x : v) x = rng.normal();
  for (auto& x : kc) x = rng.normal();
  for (auto& x : vc) x = rng.normal();
  std::vector<int32_t> slots(T);
  for (int t = 0; t < T; ++t) slots[t] = t * 37 % (nb * bs);
  slots[3] = -1;  // skipped
  slots[4] = 5 * bs;  // offset 0 of block 5: IsoQuant metadata written there
  auto dk = DeviceBuffer<float>::from_host(k), dv = DeviceBuffer<float>::from_host(v);
  auto dkc = DeviceBuffer<float>::from_host(kc), dvc = DeviceBuffer<float>::from_host(vc);
  auto dslots = DeviceBuffer<int32_t>::from_host(slots);
  std::vector<float> meta((size_t)nb * hkv * (D / 4) * 8, -7.f);
  auto dmeta = DeviceBuffer<float>::from_host(meta);
  railgun::PagedAttentionOp op(0.125f, H, hkv, D, bs, kern);
  auto cache = [&](float* p) { return TensorView::contiguous(p, DType::F32, {nb, hkv, bs, D}); };
  op.reshape_and_cache(TensorView::contiguous(dk.data(), DType::F32, {T, hkv, D}),
                       TensorView::contiguous(dv.data(), DType::F32, {T, hkv, D}), cache(dkc.data()),
                       cache(dvc.data()), dslots.data(), dmeta.data(), /*use_isoquant=*/true);
  for (int t = 0; t < T; ++t) {
    if (slots[t] < 0) continue;
    const int blk = slots[t] / bs, off = slots[t] % bs;
    for (int h = 0; h < hkv; ++h)
      for (int d = 0; d < D; ++d) {
        kc[(((size_t)blk * hkv + h) * bs + off) * D + d] = k[((size_t)t * hkv + h) * D + d];
        vc[(((size_t)blk * hkv + h) * bs + off) * D + d] = v[((size_t)t * hkv + h) * D + d];
      }
    if (off == 0)
      for (int h = 0; h < hkv; ++h)
        for (int i = 0; i < D / 4; ++i)
          for (int e = 0; e < 8; ++e) meta[(((size_t)blk * hkv + h) * (D / 4) + i) * 8 + e] = (e % 4 == 3) ? 1.f : 0.f;
  }
  require(std::memcmp(dkc.to_host().data(), kc.data(), kc.size() * 4) == 0 &&
              std::memcmp(dvc.to_host().data(), vc.data(), vc.size() * 4) == 0,
          "reshape_and_cache (IsoQuant launcher): both caches bit-exact, slot -1 skipped");
  require(std::memcmp(dmeta.to_host().data(), meta.data(), meta.size() * 4) == 0,
          "reshape_and_cache_isoquant: identity metadata at block offset 0 only");

  // apply_rope on x [T, H, D] with the HF table of the library, against host rotate-half.
  const int maxpos = 600;
  std::vector<float> table((size_t)maxpos * D);
  railgun::check(rg_rope_cos_sin_table(table.data(), maxpos, D, 500000.0), "rope table");
  std::vector<float> x((size_t)T * H * D);
  for (auto& e : x) e = rng.normal();
  std::vector<int32_t> pos(T);
  for (int t = 0; t < T; ++t) pos[t] = (t * 71) % maxpos;
  auto dx = DeviceBuffer<float>::from_host(x);
  auto dtab = DeviceBuffer<float>::from_host(table);
  auto dpos = DeviceBuffer<int32_t>::from_host(pos);
  op.apply_rope(TensorView::contiguous(dx.data(), DType::F32, {T, H, D}), dtab.data(), dpos.data());
  const std::vector<float> rx = dx.to_host();
  double worst = 0;
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < H; ++h)
      for (int i = 0; i < D / 2; ++i) {
        const double c = std::cos(pos[t] * std::pow(500000.0, -2.0 * i / D));
        const double s = std::sin(pos[t] * std::pow(500000.0, -2.0 * i / D));
        const size_t b = ((size_t)t * H + h) * D;
        const double lo = x[b + i] * c - x[b + i + D / 2] * s, hi = x[b + i + D / 2] * c + x[b + i] * s;
        worst = std::max({worst, std::fabs(lo - rx[b + i]), std::fabs(hi - rx[b + i + D / 2])});
      }
  require(worst < 1e-5, "apply_rope: rotate-half with theta 5e5 within 1e-5 of double");
}

void test_prefill(const std::shared_ptr<railgun::PagedAttentionKernels>& kern) {
  // Two sequences, one with 20 cached positions before its 37 new rows; fp32, GQA 4.
  const int H = 8, hkv = 2, D = 64, bs = 16;
  const std::vector<int32_t> lens = {45, 37}, prior = {0, 20};
  std::vector<int32_t> ctx = {lens[0] + prior[0], lens[1] + prior[1]};
  Rng rng(77);
  const int nb = 12, mb = 5;
  const std::vector<int32_t> bt = block_tables(ctx, bs, nb, mb, rng);
  std::vector<float> pool((size_t)nb * 2 * hkv * bs * D);
  for (auto& e : pool) e = rng.normal();
  const int T = lens[0] + lens[1];
  std::vector<float> q((size_t)T * H * D);
  for (auto& e : q) e = rng.normal();
  const std::vector<int32_t> cu = {0, lens[0], T};
  auto dq = DeviceBuffer<float>::from_host(q), dpool = DeviceBuffer<float>::from_host(pool);
  auto dbt = DeviceBuffer<int32_t>::from_host(bt), dctx = DeviceBuffer<int32_t>::from_host(ctx);
  auto dcu = DeviceBuffer<int32_t>::from_host(cu);
  const double scale = 0.125;
  railgun::PagedAttentionOp op((float)scale, H, hkv, D, bs, kern);
  DeviceBuffer<uint8_t> out = op.prefill_packed(
      TensorView::contiguous(dq.data(), DType::F32, {T, H, D}), pool_view(dpool.data(), DType::F32, nb, hkv, bs, D, 0),
      pool_view(dpool.data(), DType::F32, nb, hkv, bs, D, 1), TensorView::contiguous(dbt.data(), DType::F32, {2, mb}),
      TensorView::contiguous(dctx.data(), DType::F32, {2}), TensorView::contiguous(dcu.data(), DType::F32, {3}), 45);
  const std::vector<uint8_t> raw = out.to_host();
  std::vector<float> got((size_t)T * H * D);
  std::memcpy(got.data(), raw.data(), got.size() * 4);
  // Row j of sequence s is a decode with context prior_s + j + 1.
  std::vector<double> want(got.size());
  for (int s = 0; s < 2; ++s)
    for (int j = 0; j < lens[s]; ++j) {
      const int row = cu[s] + j;
      std::vector<float> qr(q.begin() + (size_t)row * H * D, q.begin() + (size_t)(row + 1) * H * D);
      const std::vector<int32_t> one_bt(bt.begin() + s * mb, bt.begin() + (s + 1) * mb);
      const std::vector<double> r = attention(qr, [&](size_t i) { return (double)pool[i]; }, one_bt,
                                              {prior[s] + j + 1}, H, hkv, D, bs, mb, scale);
      std::copy(r.begin(), r.end(), want.begin() + (size_t)row * H * D);
    }
  require(max_excess(want, got, 1e-4, 1e-4) == 0.0,
          "prefill_packed fp32: row j equals decode with context prior + j + 1 (1e-4)");
}

void test_errors(const std::shared_ptr<railgun::PagedAttentionKernels>& kern) {
  railgun::PagedAttentionOp bad(0.1f, 4, 4, 66, 16, kern);
  bool not_supported = false;
  try {
    DeviceBuffer<float> q(4 * 66);
    (void)bad.execute(TensorView::contiguous(q.data(), DType::F32, {1, 4, 66}),
                      TensorView::contiguous(q.data(), DType::F32, {1, 4, 16, 66}),
                      TensorView::contiguous(q.data(), DType::F32, {1, 4, 16, 66}),
                      TensorView::contiguous(q.data(), DType::F32, {1, 1}),
                      TensorView::contiguous(q.data(), DType::F32, {1}), nullptr, 1);
  } catch (const CoreError& e) {
    not_supported = e.kind() == CoreError::Kind::NotSupported;
  }
  require(not_supported, "execute with head_dim 66: CoreError::NotSupported");
  bool tensor_err = false;
  try {
    kern->launch_v1(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1.f, 6, 4, 64, 16, 2, 1);
  } catch (const CoreError& e) {
    tensor_err = e.kind() == CoreError::Kind::Tensor && std::strstr(e.what(), "num_kv_heads") != nullptr;
  }
  require(tensor_err, "launch_v1 with num_heads not a multiple of num_kv_heads: CoreError::Tensor");
}

}  // namespace

int main() {
  try {
    auto kern = std::make_shared<railgun::PagedAttentionKernels>(0);
    test_cache_and_rope(kern);
    test_decode(kern, DType::F32, 300, 11);
    test_decode(kern, DType::BF16, 4096, 12);
    test_decode(kern, DType::BF16, 5000, 13);
    test_prefill(kern);
    test_errors(kern);
    if (hipDeviceSynchronize() != hipSuccess) {
      std::fprintf(stderr, "FAIL: device error at exit\n");
      return 1;
    }
  } catch (const std::exception& e) {
    std::fprintf(stderr, "FAIL: unexpected exception: %s\n", e.what());
    return 1;
  }
  std::printf("all %d checks passed\n", g_checks);
  return 0;
}
