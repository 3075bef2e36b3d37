// Element-wise model operations around the attention path of a Llama decode step:
// the fused residual add + RMSNorm in front of each sublayer and the SwiGLU gate.
//
// Railgun runs these as candle ops on each layer's activations
// (crates/vllm-models/src/llama/architecture.rs:38-59 and :80-84): RmsNorm computes in
// fp32 and rounds once to the activation dtype; `x + residual` and `silu(gate) * up` are
// element-wise ops whose every result is rounded to the activation dtype.  Both kernels
// keep those roundings: rows are [hidden] contiguous, one workgroup per row, 16-byte
// vector moves where the row and pointers allow (they are HBM-bound).
#include <math.h>

#include "rg_common.hpp"

namespace rg {
namespace {

constexpr int kRowThreads = 256;

// Sum over a 256-thread workgroup (wave shuffles, then 4 partials through LDS).
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // `red` is free (an earlier call's readers are done)
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// residual != nullptr:  residual <- round(residual + x);  out <- round(rms(residual) * w)
// residual == nullptr:  out <- round(rms(x) * w)
// rms(r) = r / sqrt(mean(r^2) + eps), computed in fp32 on the rounded sum.
template <typename T>
__global__ __launch_bounds__(kRowThreads) void rms_norm_kernel(const typename elem<T>::storage* __restrict__ x,
                                                               typename elem<T>::storage* __restrict__ residual,
                                                               const typename elem<T>::storage* __restrict__ w,
                                                               typename elem<T>::storage* __restrict__ out,
                                                               float eps, int hidden) {
  using E = elem<T>;
  using S = typename E::storage;
  __shared__ float red[kRowThreads / 64];
  const int64_t base = (int64_t)blockIdx.x * hidden;
  const S* xr = x + base;
  S* rr = residual ? residual + base : nullptr;
  float ss = 0.f;
  for (int i = threadIdx.x; i < hidden; i += kRowThreads) {
    float v = E::to_f32(xr[i]);
    if (rr) {
      const S sum = E::from_f32(E::to_f32(rr[i]) + v);
      rr[i] = sum;
      v = E::to_f32(sum);
    }
    ss += v * v;
  }
  const float inv = rsqrtf(block_sum(ss, red) / (float)hidden + eps);
  const S* src = rr ? rr : xr;
  S* o = out + base;
  for (int i = threadIdx.x; i < hidden; i += kRowThreads) {
    o[i] = E::from_f32(E::to_f32(src[i]) * inv * E::to_f32(w[i]));
  }
}

// 16-bit dtypes with hidden % 8 == 0 and 16-byte aligned rows: each thread moves 8 values
// per step.
template <typename T>
__global__ __launch_bounds__(kRowThreads) void rms_norm_vec8_kernel(const uint4* __restrict__ x,
                                                                    uint4* __restrict__ residual,
                                                                    const uint4* __restrict__ w,
                                                                    uint4* __restrict__ out, float eps,
                                                                    int hidden) {
  using E = elem<T>;
  __shared__ float red[kRowThreads / 64];
  const int nv = hidden / 8;
  const int64_t base = (int64_t)blockIdx.x * nv;
  auto unpack = [](uint4 u, float* f) {
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = E::to_f32((uint16_t)(wd[i] & 0xffffu));
      f[2 * i + 1] = E::to_f32((uint16_t)(wd[i] >> 16));
    }
  };
  auto pack = [](const float* f) {
    uint32_t wd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wd[i] = (uint32_t)E::from_f32(f[2 * i]) | ((uint32_t)E::from_f32(f[2 * i + 1]) << 16);
    return make_uint4(wd[0], wd[1], wd[2], wd[3]);
  };
  float ss = 0.f;
  for (int i = threadIdx.x; i < nv; i += kRowThreads) {
    float v[8];
    unpack(x[base + i], v);
    if (residual) {
      float r[8];
      unpack(residual[base + i], r);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] += v[e];
      const uint4 sum = pack(r);
      residual[base + i] = sum;
      unpack(sum, v);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  }
  const float inv = rsqrtf(block_sum(ss, red) / (float)hidden + eps);
  const uint4* src = residual ? residual : x;
  for (int i = threadIdx.x; i < nv; i += kRowThreads) {
    float v[8], g[8];
    unpack(src[base + i], v);
    unpack(w[i], g);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = v[e] * inv * g[e];
    out[base + i] = pack(v);
  }
}

// out[r, i] = round(round(silu(g)) * u) with g = gate_up[r, i], u = gate_up[r, inter + i]
// (candle: silu(gate_proj(x)) * up_proj(x), each op rounded to the activation dtype).
template <typename T>
__global__ __launch_bounds__(kRowThreads) void silu_mul_kernel(const typename elem<T>::storage* __restrict__ gu,
                                                               typename elem<T>::storage* __restrict__ out,
                                                               int inter) {
  using E = elem<T>;
  const int64_t r = blockIdx.y;
  const int i = blockIdx.x * kRowThreads + threadIdx.x;
  if (i >= inter) return;
  const float g = E::to_f32(gu[r * 2 * inter + i]);
  const float u = E::to_f32(gu[r * 2 * inter + inter + i]);
  const float a = E::to_f32(E::from_f32(g / (1.f + expf(-g))));
  out[r * inter + i] = E::from_f32(a * u);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace rg

using namespace rg;

extern "C" int rg_rms_norm(const void* x, void* residual, const void* weight, void* out, float eps,
                           int32_t num_rows, int32_t hidden_size, int32_t dtype, void* stream) {
  const char* op = "rms_norm";
  if (dtype_bytes(dtype) == 0) return fail(RG_ERR_NOT_SUPPORTED, "%s: unknown dtype %d", op, dtype);
  if (num_rows < 0 || hidden_size <= 0) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: need num_rows >= 0 and hidden_size > 0 (got %d, %d)", op, num_rows,
                hidden_size);
  }
  if (!(eps >= 0.f)) return fail(RG_ERR_INVALID_ARGUMENT, "%s: eps must be >= 0", op);
  if (num_rows == 0) return ok();
  if (!x || !weight || !out) return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  hipStream_t s = as_stream(stream);
  const bool vec = dtype != RG_DTYPE_F32 && hidden_size % 8 == 0 && aligned16(x) && aligned16(weight) &&
                   aligned16(out) && (residual == nullptr || aligned16(residual));
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    using S = typename elem<T>::storage;
    if constexpr (!std::is_same_v<T, f32_t>) {
      if (vec) {
        hipLaunchKernelGGL(rms_norm_vec8_kernel<T>, dim3(num_rows), dim3(kRowThreads), 0, s,
                           static_cast<const uint4*>(x), static_cast<uint4*>(residual),
                           static_cast<const uint4*>(weight), static_cast<uint4*>(out), eps, hidden_size);
        return check_launch(op);
      }
    }
    hipLaunchKernelGGL(rms_norm_kernel<T>, dim3(num_rows), dim3(kRowThreads), 0, s, static_cast<const S*>(x),
                       static_cast<S*>(residual), static_cast<const S*>(weight), static_cast<S*>(out), eps,
                       hidden_size);
    return check_launch(op);
  });
}

extern "C" int rg_silu_and_mul(const void* gate_up, void* out, int32_t num_rows, int32_t intermediate_size,
                               int32_t dtype, void* stream) {
  const char* op = "silu_and_mul";
  if (dtype_bytes(dtype) == 0) return fail(RG_ERR_NOT_SUPPORTED, "%s: unknown dtype %d", op, dtype);
  if (num_rows < 0 || intermediate_size <= 0 || num_rows > 65535) {
    return fail(RG_ERR_INVALID_ARGUMENT, "%s: need 0 <= num_rows <= 65535 and intermediate_size > 0 (got %d, %d)",
                op, num_rows, intermediate_size);
  }
  if (num_rows == 0) return ok();
  if (!gate_up || !out) return fail(RG_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)ceil_div(intermediate_size, kRowThreads), (unsigned)num_rows);
  return dispatch_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    using S = typename elem<T>::storage;
    hipLaunchKernelGGL(silu_mul_kernel<T>, grid, dim3(kRowThreads), 0, s, static_cast<const S*>(gate_up),
                       static_cast<S*>(out), intermediate_size);
    return check_launch(op);
  });
}
