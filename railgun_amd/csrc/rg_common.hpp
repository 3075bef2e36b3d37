// Shared device/host helpers for the gfx950 kernels of the attention hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "railgun_hip.h"

namespace rg {

// ---------------------------------------------------------------- status ----

// Records `msg` (printf-style) as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread's last error and returns RG_OK.
int ok();

// Converts a launch's hipError_t (hipGetLastError) into a status code.
int check_launch(const char* what);
// Compute units of the current device (256 if the query fails).
int device_cu_count();

// ------------------------------------------------------------ element types --

// Storage types: fp32, bf16 and fp16 are all handled as their bit patterns.
struct f32_t { using storage = float; };
struct bf16_t { using storage = uint16_t; };
struct f16_t { using storage = uint16_t; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t bits) {
  _Float16 h = __builtin_bit_cast(_Float16, bits);
  return (float)h;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

// RoPE (rotate-half) of one pair (lo, hi) = (x[i], x[i + D/2]) with the rounding of the
// reference expression (rope.cu:34-41) made explicit: each product and the difference / sum
// rounded separately (no fused multiply-add), so every kernel that rotates gets the same bits.
__device__ __forceinline__ void rope_rotate_pair(float lo, float hi, float c, float s, float& out_lo,
                                                 float& out_hi) {
#pragma clang fp contract(off)
  const float a = lo * c;
  const float b = hi * s;
  const float e = hi * c;
  const float f = lo * s;
  out_lo = a - b;
  out_hi = e + f;
}

template <typename T> struct elem;
template <> struct elem<f32_t> {
  using storage = float;
  static constexpr int bytes = 4;
  __device__ static __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  __device__ static __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
  __device__ static __forceinline__ float to_f32(float v) { return v; }
  __device__ static __forceinline__ float from_f32(float v) { return v; }
};
template <> struct elem<bf16_t> {
  using storage = uint16_t;
  static constexpr int bytes = 2;
  __device__ static __forceinline__ float load(const uint16_t* p, int64_t i) {
    return bf16_bits_to_f32(p[i]);
  }
  __device__ static __forceinline__ void store(uint16_t* p, int64_t i, float v) {
    p[i] = f32_to_bf16_bits(v);
  }
  __device__ static __forceinline__ float to_f32(uint16_t v) { return bf16_bits_to_f32(v); }
  __device__ static __forceinline__ uint16_t from_f32(float v) { return f32_to_bf16_bits(v); }
};
template <> struct elem<f16_t> {
  using storage = uint16_t;
  static constexpr int bytes = 2;
  __device__ static __forceinline__ float load(const uint16_t* p, int64_t i) {
    return f16_bits_to_f32(p[i]);
  }
  __device__ static __forceinline__ void store(uint16_t* p, int64_t i, float v) {
    p[i] = f32_to_f16_bits(v);
  }
  __device__ static __forceinline__ float to_f32(uint16_t v) { return f16_bits_to_f32(v); }
  __device__ static __forceinline__ uint16_t from_f32(float v) { return f32_to_f16_bits(v); }
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
// Two values rounded to nearest even and packed into one word, low half first
// (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
template <typename T> __device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <> __device__ __forceinline__ uint32_t pack2<bf16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});
}
template <> __device__ __forceinline__ uint32_t pack2<f16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, f16x2_t{(_Float16)lo, (_Float16)hi});
}

inline int dtype_bytes(int32_t dtype) {
  switch (dtype) {
    case RG_DTYPE_F32: return 4;
    case RG_DTYPE_BF16: return 2;
    case RG_DTYPE_F16: return 2;
    default: return 0;
  }
}

inline const char* dtype_name(int32_t dtype) {
  switch (dtype) {
    case RG_DTYPE_F32: return "f32";
    case RG_DTYPE_BF16: return "bf16";
    case RG_DTYPE_F16: return "f16";
    default: return "?";
  }
}

// Calls f(tag) with tag = f32_t / bf16_t / f16_t for the runtime dtype.
template <typename F>
inline int dispatch_dtype(int32_t dtype, F&& f) {
  switch (dtype) {
    case RG_DTYPE_F32: return f(f32_t{});
    case RG_DTYPE_BF16: return f(bf16_t{});
    case RG_DTYPE_F16: return f(f16_t{});
    default: return fail(RG_ERR_NOT_SUPPORTED, "unknown dtype code %d", (int)dtype);
  }
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// ------------------------------------------------------- wave-level helpers --

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}


// ------------------------------------------------------- streamed loads --

typedef unsigned rg_u32x4_t __attribute__((ext_vector_type(4)));
// 16 bytes read once per call (paged K/V rows): a non-temporal load (the `nt` bit), so the
// line streams through the caches instead of being kept for reuse.  Measured on the stream-K
// decode at config 2: 113.3 -> 97.6 us per call, same results.  Only where the instructions
// that share a cache line are issued together: the fp32 decode tile, whose eight K loads of a
// lane cover one line in 16-byte steps, ran 1.6x slower with it on K (it keeps it on V), and
// the prefill's tile copies, which later units of the same kv-head re-read, 12 % slower.
__device__ __forceinline__ uint4 stream_load16(const void* p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(static_cast<const rg_u32x4_t*>(p)));
}

// ------------------------------------------------------------ LDS staging --

#define RG_LDS __attribute__((address_space(3)))

// 16 bytes per lane from global memory straight into LDS at lds_addr + 16 * lane (the
// vector memory counter tracks completion).  Issued through asm so that the compiler does
// not add a full vector-memory wait in front of every LDS read; each kernel orders the
// copies itself with an explicit vmcnt wait + tile_barrier.
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr) : "memory", "m0");
}
// The same copy from a wave-uniform base plus a 32-bit per-lane byte offset.
__device__ __forceinline__ void lds_dma16_s(const char* base, uint32_t lane_bytes, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(lane_bytes), "s"(base), "s"(lds_addr)
               : "memory", "m0");
}
// lds_dma16_s for data read once per call (GEMM weights): non-temporal (`nt`), as
// stream_load16.  Measured on the decode-step projections: 5-10 % faster at 1 row, 1-4 % at 128.
__device__ __forceinline__ void lds_dma16_s_nt(const char* base, uint32_t lane_bytes, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(lane_bytes), "s"(base), "s"(lds_addr)
               : "memory", "m0");
}
// Workgroup barrier without the memory fence of __syncthreads (which would also wait for
// every prefetch in flight); the asm statements keep the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void tile_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace rg
