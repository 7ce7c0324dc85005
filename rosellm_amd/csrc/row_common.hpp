// Pieces shared by the log-prob row kernels: element tags, row alignment split,
// online (max, sum-exp) accumulation and the dlogits sweep.
#pragma once

#include "rrl_common.hpp"

namespace rrl {

struct RowArgs {
  const void* logits;
  int64_t B, T, V, ls_b, ls_t;
  View tgt;
  // forward outputs
  void* logp;
  int logp_dt;
  void* lse_out;
  // backward inputs (logp_in may be null: the target column then uses lse)
  const void* lse;
  const void* g;
  const void* logp_in;
  // dlogits
  void* dl;
  int dl_dt;
  int64_t ds_b, ds_t;
  int accumulate;
  // single pass
  rrl_policy_params pp;
  View old, adv, mask;
  const void* row_coef;
  void* records;  // register-resident path: packed per-token records (TokenRecord)
  int32_t* status;
};

// One token's inputs to the single-pass kernel, packed for a single 16-byte
// scalar load per row: target id (-1 when outside [0, V)), old log-prob,
// advantage and mask weight * row coefficient.
struct TokenRecord {
  int32_t target;
  float old;
  float adv;
  float wcoef;
};

__device__ __forceinline__ int dtype_size_dev(int dt) {
  return dt == RRL_F64 ? 8 : (dt == RRL_F32 ? 4 : 2);
}

// Element tags: storage type, accumulation type, elements per 16-byte vector.
struct TagBF16 {
  using S = uint16_t;
  using Acc = float;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float cvt(uint16_t v) { return bf16_bits_to_f32(v); }
  static __device__ __forceinline__ void load_vec(const uint16_t* p, float (&x)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    x[0] = __uint_as_float(u.x << 16); x[1] = __uint_as_float(u.x & 0xffff0000u);
    x[2] = __uint_as_float(u.y << 16); x[3] = __uint_as_float(u.y & 0xffff0000u);
    x[4] = __uint_as_float(u.z << 16); x[5] = __uint_as_float(u.z & 0xffff0000u);
    x[6] = __uint_as_float(u.w << 16); x[7] = __uint_as_float(u.w & 0xffff0000u);
  }
};
struct TagF16 {
  using S = uint16_t;
  using Acc = float;
  static constexpr int VEC = 8;
  static __device__ __forceinline__ float cvt(uint16_t v) { return f16_bits_to_f32(v); }
  static __device__ __forceinline__ void load_vec(const uint16_t* p, float (&x)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = f16_bits_to_f32((uint16_t)(w[i] & 0xffffu));
      x[2 * i + 1] = f16_bits_to_f32((uint16_t)(w[i] >> 16));
    }
  }
};
struct TagF32 {
  using S = float;
  using Acc = float;
  static constexpr int VEC = 4;
  static __device__ __forceinline__ float cvt(float v) { return v; }
  static __device__ __forceinline__ void load_vec(const float* p, float (&x)[4]) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
  }
};
struct TagF64 {
  using S = double;
  using Acc = double;
  static constexpr int VEC = 2;
  static __device__ __forceinline__ double cvt(double v) { return v; }
  static __device__ __forceinline__ void load_vec(const double* p, double (&x)[2]) {
    const double2 u = *reinterpret_cast<const double2*>(p);
    x[0] = u.x; x[1] = u.y;
  }
};

// A row of V elements split into a scalar head (up to the first 16-byte
// boundary), a body of whole 16-byte vectors and a scalar tail.
struct RowSplit {
  int64_t head, nvec, tail;
  template <typename S, int VEC>
  __device__ __forceinline__ static RowSplit make(const S* row, int64_t V) {
    RowSplit r;
    const uintptr_t mis = reinterpret_cast<uintptr_t>(row) & 15u;
    int64_t h = mis ? (int64_t)((16u - mis) / sizeof(S)) : 0;
    if (h > V) h = V;
    r.head = h;
    r.nvec = (V - h) / VEC;
    r.tail = V - h - r.nvec * VEC;
    return r;
  }
};

// exp(x - m) for the online accumulator.
template <typename Acc>
__device__ __forceinline__ Acc exp_diff(Acc x, Acc m) { return M<Acc>::fast_exp(x - m); }

// Fold N new values into a running (max, sum exp(x - max)).  The max covers
// every value; element `skip` (the target column, or -1 for none) is left out
// of the sum so that the target's log-prob can be formed without cancellation
// (finish_row).  Values equal to -inf contribute zero; NaN reaches the sum
// through exp.
template <typename Acc, int N>
__device__ __forceinline__ void online_update(Acc& m, Acc& s, const Acc (&x)[N], int skip) {
  Acc mc = x[0];
#pragma unroll
  for (int i = 1; i < N; ++i) mc = fmax(mc, x[i]);
  if (mc > m) {
    s = s * exp_diff<Acc>(m, mc);
    m = mc;
  }
  if (m != -M<Acc>::inf()) {
    if (skip < 0) {
#pragma unroll
      for (int i = 0; i < N; ++i) s += exp_diff<Acc>(x[i], m);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) s += (i == skip) ? Acc(0) : exp_diff<Acc>(x[i], m);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (x[i] != x[i] && i != skip) s += x[i];
  }
}

// Row log-sum-exp and target log-prob from the row max M (over all columns),
// S_other = sum over the non-target columns of exp(x - M), and the target
// logit xt.  With e_t = exp(xt - M):
//   lse  = M + log(S_other + e_t)
//   logp = -log1p(S_other / e_t)          when xt is within 1 of the max,
//          (xt - M) - log(S_other + e_t)  otherwise.
// The first form keeps full relative precision as logp -> 0 (a dominant
// target), where xt - lse would cancel.  An all -inf row gives NaN, as
// log_softmax does; NaN or +inf anywhere in the row gives NaN.
template <typename Acc>
struct RowLogprob {
  Acc lse, logp;
};

template <typename Acc>
__device__ __forceinline__ RowLogprob<Acc> finish_row(Acc Mx, Acc S_other, Acc xt) {
  // Branch-free: both forms are evaluated and selected, which keeps the
  // results in registers.
  const bool empty = Mx == -M<Acc>::inf();
  const Acc dt = xt - Mx;
  const Acc et = M<Acc>::exp(dt);
  const Acc S = S_other + et;
  const Acc lse = Mx + M<Acc>::log(S);
  const Acc near = -M<Acc>::log1p(S_other / et);
  const Acc far = dt - M<Acc>::log(S);
  RowLogprob<Acc> r;
  r.lse = empty ? -M<Acc>::inf() : ((S != S) ? M<Acc>::nan() : lse);
  r.logp = empty ? M<Acc>::nan() : ((dt > Acc(-1)) ? near : far);
  return r;
}

template <typename Acc>
__device__ __forceinline__ void online_merge(Acc& m, Acc& s, Acc m2, Acc s2) {
  const Acc mn = fmax(m, m2);
  if (mn == -M<Acc>::inf()) {
    s = s + s2;
  } else {
    s = s * exp_diff<Acc>(m, mn) + s2 * exp_diff<Acc>(m2, mn);
  }
  m = mn;
}

// Combine the per-lane (m, s) over the workgroup; every thread gets the total.
template <int NT, typename Acc>
__device__ __forceinline__ void block_online_combine(Acc& m, Acc& s, Acc* sh_m, Acc* sh_s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const Acc m2 = __shfl_xor(m, o, 64);
    const Acc s2 = __shfl_xor(s, o, 64);
    online_merge(m, s, m2, s2);
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    sh_m[w] = m;
    sh_s[w] = s;
  }
  __syncthreads();
  m = sh_m[0];
  s = sh_s[0];
  for (int i = 1; i < NT / 64; ++i) online_merge(m, s, sh_m[i], sh_s[i]);
  __syncthreads();
}

// Store N consecutive gradient values at element offset `col` of an output row.
template <typename Acc, int N>
__device__ __forceinline__ void store_run(void* drow, int dt, int64_t col, const Acc (&d)[N],
                                          bool vec_ok) {
  if (dt == RRL_BF16 && vec_ok && (N % 2) == 0) {
    uint32_t w[N / 2 > 0 ? N / 2 : 1];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) w[i] = f32x2_to_bf16x2_bits((float)d[2 * i], (float)d[2 * i + 1]);
    uint16_t* p = static_cast<uint16_t*>(drow) + col;
    if (N == 8) {
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[N > 2 ? 1 : 0], w[N > 4 ? 2 : 0], w[N > 6 ? 3 : 0]);
    } else if (N == 4) {
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[N > 2 ? 1 : 0]);
    } else {
      *reinterpret_cast<uint32_t*>(p) = w[0];
    }
    return;
  }
  if (dt == RRL_F32 && vec_ok && (N % 4) == 0) {
    float* p = static_cast<float*>(drow) + col;
#pragma unroll
    for (int i = 0; i < N; i += 4)
      *reinterpret_cast<float4*>(p + i) = make_float4((float)d[i], (float)d[i + 1], (float)d[i + 2], (float)d[i + 3]);
    return;
  }
#pragma unroll
  for (int i = 0; i < N; ++i) store_as<Acc>(drow, dt, col + i, d[i]);
}

// Sweep 2 over one row: d[v] = -g * exp(x[v] - lse) for v != target and
// d[target] = tgt_d, the composition of gather's and log_softmax's backward
// (losses.py:34-38).  The caller forms tgt_d = g * (1 - p_target) as
// -g * expm1(logp) so that it keeps its relative precision when p_target -> 1.
// zero_row skips reading the logits (g == 0 and a finite lse give exact zeros).
template <class Tag, int NT>
__device__ __forceinline__ void write_row_grad(const typename Tag::S* row, const RowSplit& sp,
                                               void* drow, int dl_dt, int64_t V, int64_t target,
                                               typename Tag::Acc g, typename Tag::Acc lse,
                                               typename Tag::Acc tgt_d, bool zero_row,
                                               int accumulate) {
  using Acc = typename Tag::Acc;
  constexpr int VEC = Tag::VEC;
  const int osz = dtype_size_dev(dl_dt);
  const uintptr_t body_addr = reinterpret_cast<uintptr_t>(drow) + (uintptr_t)(sp.head * osz);
  const int need = (VEC * osz) < 16 ? (VEC * osz) : 16;
  const bool vec_ok = !accumulate && (body_addr % (uintptr_t)need) == 0;

  auto elem = [&](int64_t col, Acc x) -> Acc {
    Acc d = (col == target) ? tgt_d : -(M<Acc>::fast_exp(x - lse) * g);
    if (accumulate) d += load_as<Acc>(drow, dl_dt, col);
    return d;
  };

  for (int64_t i = threadIdx.x; i < sp.head; i += NT) {
    Acc d[1] = {zero_row ? Acc(0) : elem(i, Tag::cvt(row[i]))};
    store_run<Acc, 1>(drow, dl_dt, i, d, false);
  }
  const typename Tag::S* body = row + sp.head;
  for (int64_t k = threadIdx.x; k < sp.nvec; k += NT) {
    const int64_t col0 = sp.head + k * VEC;
    Acc d[VEC];
    if (zero_row) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) d[i] = Acc(0);
    } else {
      Acc x[VEC];
      Tag::load_vec(body + k * VEC, x);
#pragma unroll
      for (int i = 0; i < VEC; ++i) d[i] = elem(col0 + i, x[i]);
    }
    store_run<Acc, VEC>(drow, dl_dt, col0, d, vec_ok);
  }
  const int64_t tail0 = sp.head + sp.nvec * VEC;
  for (int64_t i = threadIdx.x; i < sp.tail; i += NT) {
    Acc d[1] = {zero_row ? Acc(0) : elem(tail0 + i, Tag::cvt(row[tail0 + i]))};
    store_run<Acc, 1>(drow, dl_dt, tail0 + i, d, false);
  }
}

// Target-column gradient g * (1 - p_target).  With the row's log-prob at hand
// it is -g * expm1(logp); otherwise it falls back to g - g * exp(xt - lse).
template <typename Acc>
__device__ __forceinline__ Acc target_grad(Acc g, Acc logp, bool have_logp, Acc xt, Acc lse) {
  if (have_logp) return -(g * M<Acc>::expm1(logp));
  return g - M<Acc>::exp(xt - lse) * g;
}

}  // namespace rrl
