// Shared device/host helpers for the gfx950 kernels: dtype-dispatched loads
// and stores over strided views, wave64/workgroup reductions, error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "roserlhf_amd.h"

namespace rrl {

// ---------------------------------------------------------------------------
// Host-side error handling.  Each entry point returns an rrl_status and leaves a
// per-thread message behind.
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
void clear_error();

#define RRL_REQUIRE(cond, code, msg)        \
  do {                                      \
    if (!(cond)) {                          \
      ::rrl::set_error(msg);                \
      return (code);                        \
    }                                       \
  } while (0)

int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool is_float_dtype(int dt) {
  return dt == RRL_F32 || dt == RRL_F64 || dt == RRL_BF16 || dt == RRL_F16;
}
inline bool is_known_dtype(int dt) { return dt >= RRL_F32 && dt <= RRL_I64; }
inline size_t dtype_size(int dt) {
  switch (dt) {
    case RRL_F32: return 4;
    case RRL_F64: return 8;
    case RRL_BF16:
    case RRL_F16:
    case RRL_I16: return 2;
    case RRL_BOOL:
    case RRL_U8:
    case RRL_I8: return 1;
    case RRL_I32: return 4;
    case RRL_I64: return 8;
    default: return 0;
  }
}

// ---------------------------------------------------------------------------
// Device-side scalar conversions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
// Round-to-nearest-even float -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  f2 v = {x, x};
  b2 r = __builtin_convertvector(v, b2);
  return (uint16_t)(__builtin_bit_cast(uint32_t, r) & 0xffffu);
}
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  f2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// Load element i of an array of dtype `dt` converted to Acc.  `dt` is uniform
// across the wave, so the switch is a scalar branch.
template <typename Acc>
__device__ __forceinline__ Acc load_as(const void* p, int dt, int64_t i) {
  switch (dt) {
    case RRL_F32: return (Acc)(static_cast<const float*>(p)[i]);
    case RRL_F64: return (Acc)(static_cast<const double*>(p)[i]);
    case RRL_BF16: return (Acc)bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    case RRL_F16: return (Acc)f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    case RRL_BOOL:
    case RRL_U8: return (Acc)(static_cast<const uint8_t*>(p)[i]);
    case RRL_I8: return (Acc)(static_cast<const int8_t*>(p)[i]);
    case RRL_I16: return (Acc)(static_cast<const int16_t*>(p)[i]);
    case RRL_I32: return (Acc)(static_cast<const int32_t*>(p)[i]);
    case RRL_I64: return (Acc)(static_cast<const int64_t*>(p)[i]);
    default: return (Acc)0;
  }
}

// Truth value of element i (torch .to(bool): nonzero, NaN counts as true).
__device__ __forceinline__ bool load_bool(const void* p, int dt, int64_t i) {
  switch (dt) {
    case RRL_F32: return static_cast<const float*>(p)[i] != 0.0f;
    case RRL_F64: return static_cast<const double*>(p)[i] != 0.0;
    case RRL_BF16:
    case RRL_F16: return (static_cast<const uint16_t*>(p)[i] & 0x7fffu) != 0;
    case RRL_BOOL:
    case RRL_U8:
    case RRL_I8: return static_cast<const uint8_t*>(p)[i] != 0;
    case RRL_I16: return static_cast<const int16_t*>(p)[i] != 0;
    case RRL_I32: return static_cast<const int32_t*>(p)[i] != 0;
    case RRL_I64: return static_cast<const int64_t*>(p)[i] != 0;
    default: return false;
  }
}

__device__ __forceinline__ int64_t load_index(const void* p, int dt, int64_t i) {
  return dt == RRL_I32 ? (int64_t)(static_cast<const int32_t*>(p)[i])
                       : static_cast<const int64_t*>(p)[i];
}

template <typename Acc>
__device__ __forceinline__ void store_as(void* p, int dt, int64_t i, Acc v) {
  switch (dt) {
    case RRL_F32: static_cast<float*>(p)[i] = (float)v; break;
    case RRL_F64: static_cast<double*>(p)[i] = (double)v; break;
    case RRL_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits((float)v); break;
    case RRL_F16: static_cast<uint16_t*>(p)[i] = f32_to_f16_bits((float)v); break;
    default: break;
  }
}

// Strided [rows, cols] operand.
struct View {
  const void* ptr;
  int dt;
  int64_t sr, sc;
  __host__ __device__ bool present() const { return ptr != nullptr; }
  template <typename Acc>
  __device__ __forceinline__ Acc get(int64_t r, int64_t c) const {
    return load_as<Acc>(ptr, dt, r * sr + c * sc);
  }
  __device__ __forceinline__ bool truth(int64_t r, int64_t c) const {
    return load_bool(ptr, dt, r * sr + c * sc);
  }
};
inline View to_view(const rrl_view& v) { return View{v.ptr, v.dtype, v.s_row, v.s_col}; }

// ---------------------------------------------------------------------------
// Math helpers, float and double.
// ---------------------------------------------------------------------------
template <typename T> struct M;
template <> struct M<float> {
  static __device__ __forceinline__ float exp(float x) { return expf(x); }
  static __device__ __forceinline__ float log(float x) { return logf(x); }
  static __device__ __forceinline__ float log1p(float x) { return log1pf(x); }
  static __device__ __forceinline__ float expm1(float x) { return expm1f(x); }
  // v_exp_f32-based; used in the vocabulary sweeps where ~2 ulp is ample.
  static __device__ __forceinline__ float fast_exp(float x) { return __expf(x); }
  static __device__ __forceinline__ float sqrt(float x) { return __fsqrt_rn(x); }
  static __device__ __forceinline__ float inf() { return __builtin_huge_valf(); }
  static __device__ __forceinline__ float nan() { return __builtin_nanf(""); }
};
template <> struct M<double> {
  static __device__ __forceinline__ double exp(double x) { return ::exp(x); }
  static __device__ __forceinline__ double fast_exp(double x) { return ::exp(x); }
  static __device__ __forceinline__ double log(double x) { return ::log(x); }
  static __device__ __forceinline__ double log1p(double x) { return ::log1p(x); }
  static __device__ __forceinline__ double expm1(double x) { return ::expm1(x); }
  static __device__ __forceinline__ double sqrt(double x) { return ::sqrt(x); }
  static __device__ __forceinline__ double inf() { return __builtin_huge_val(); }
  static __device__ __forceinline__ double nan() { return __builtin_nan(""); }
};

// torch.clamp(x, lo, hi): NaN propagates.
template <typename T>
__device__ __forceinline__ T clampt(T x, T lo, T hi) {
  return x != x ? x : (x < lo ? lo : (x > hi ? hi : x));
}
// d clamp(x, lo, hi) / dx : gradient passes on the closed interval.
template <typename T>
__device__ __forceinline__ T clamp_pass(T x, T lo, T hi) {
  return (x >= lo && x <= hi) ? T(1) : T(0);
}
// torch.minimum(a, b) with its backward split: returns min and the share of the
// upstream gradient routed to a (1, 0 or 1/2 on ties); b gets 1 - share.
template <typename T>
__device__ __forceinline__ T min_with_share(T a, T b, T& share_a) {
  if (a < b) { share_a = T(1); return a; }
  if (b < a) { share_a = T(0); return b; }
  share_a = T(0.5);
  return (a != a) ? a : b;
}

// ---------------------------------------------------------------------------
// Reductions (wave64 shuffles, LDS across waves).  Deterministic: the order of
// combination depends only on the launch shape.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum K values over a workgroup of NT threads; every thread gets the totals.
// `sh` must hold NT/64 * K elements.
template <int NT, int K, typename T>
__device__ __forceinline__ void block_sum(T (&v)[K], T* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = wave_sum(v[k]);
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) sh[w * K + k] = v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) {
    T s = T(0);
    for (int i = 0; i < NT / 64; ++i) s += sh[i * K + k];
    v[k] = s;
  }
  __syncthreads();
}

__device__ __forceinline__ void raise_flag(int32_t* status, int32_t bit) {
  if (status) atomicOr(status, bit);
}

}  // namespace rrl
