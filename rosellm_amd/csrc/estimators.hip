// Return and advantage estimators (advantages.py:25-290), masked reductions
// (losses.py:41-50, :104-124, :489-512) and masked whitening.
//
// The reverse recurrences (discounted returns, GAE, skip-observation GAE) are
// affine maps on a small carried state, with padding acting as the identity.
// One workgroup owns one sequence; each lane owns a contiguous chunk of time
// steps:
//   1. every lane composes the affine map of its chunk (reverse time);
//   2. a log-depth suffix scan of the chunk maps over the lanes (8 steps
//      through LDS for 256 lanes) gives each lane the composition of every
//      later chunk, hence its chunk's incoming state;
//   3. every lane replays its chunk with the reference's step arithmetic from
//      its incoming state and writes the outputs.
#include "rrl_common.hpp"

namespace rrl {

namespace {

constexpr int SCAN_NT = 256;

struct ScanArgs {
  int64_t B, T;
  View r, v, nv;      // rewards, values / action_end_values, next_action_values
  View term, valid;   // optional (ptr == nullptr)
  View boot;          // optional [B]
  double gamma, lam;
  void* out0;         // returns / advantages
  void* out1;         // value targets
  int odt;
};

// Affine map on a D-dimensional state: S' = Mx * S + c (row-major Mx).
template <typename Acc, int D>
struct Aff {
  Acc m[D * D];
  Acc c[D];
  __device__ __forceinline__ static Aff identity() {
    Aff a;
#pragma unroll
    for (int i = 0; i < D * D; ++i) a.m[i] = Acc(0);
#pragma unroll
    for (int i = 0; i < D; ++i) { a.m[i * D + i] = Acc(1); a.c[i] = Acc(0); }
    return a;
  }
  // this <- step o this  (apply `this` first, then step)
  __device__ __forceinline__ void prepend(const Aff& s) {
    Aff r;
#pragma unroll
    for (int i = 0; i < D; ++i) {
#pragma unroll
      for (int j = 0; j < D; ++j) {
        Acc acc = Acc(0);
#pragma unroll
        for (int k = 0; k < D; ++k) acc += s.m[i * D + k] * m[k * D + j];
        r.m[i * D + j] = acc;
      }
      Acc acc = s.c[i];
#pragma unroll
      for (int k = 0; k < D; ++k) acc += s.m[i * D + k] * c[k];
      r.c[i] = acc;
    }
    *this = r;
  }
  __device__ __forceinline__ void apply(Acc (&S)[D]) const {
    Acc o[D];
#pragma unroll
    for (int i = 0; i < D; ++i) {
      Acc acc = c[i];
#pragma unroll
      for (int k = 0; k < D; ++k) acc += m[i * D + k] * S[k];
      o[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < D; ++i) S[i] = o[i];
  }
};

// Per-estimator step definitions.  KIND 0: discounted returns (state R).
// KIND 1: GAE (state next_value, next_advantage).  KIND 2: skip-observation
// GAE (state next_advantage).
template <int KIND> struct StateDim { static constexpr int D = KIND == 1 ? 2 : 1; };

template <typename Acc, int KIND>
__device__ __forceinline__ Aff<Acc, StateDim<KIND>::D> step_map(const ScanArgs& a, int64_t b,
                                                              int64_t t, Acc g, Acc gl) {
  constexpr int D = StateDim<KIND>::D;
  Aff<Acc, D> f = Aff<Acc, D>::identity();
  const bool valid = a.valid.present() ? a.valid.truth(b, t) : true;
  if (!valid) return f;
  const Acc nt = (a.term.present() && a.term.truth(b, t)) ? Acc(0) : Acc(1);
  if (KIND == 0) {
    f.m[0] = g * nt;
    f.c[0] = a.r.get<Acc>(b, t);
  } else if (KIND == 1) {
    const Acc V = a.v.get<Acc>(b, t);
    f.m[0] = Acc(0); f.m[1] = Acc(0);
    f.m[2] = g * nt; f.m[3] = gl * nt;
    f.c[0] = V;
    f.c[1] = a.r.get<Acc>(b, t) - V;
  } else {
    f.m[0] = gl * nt;
    f.c[0] = (a.r.get<Acc>(b, t) + (g * nt) * a.nv.get<Acc>(b, t)) - a.v.get<Acc>(b, t);
  }
  return f;
}

// Reference step (advantages.py:75-79, :129-139, :196-210): update the state
// in place and return the outputs for time t.
template <typename Acc, int KIND>
__device__ __forceinline__ void ref_step(const ScanArgs& a, int64_t b, int64_t t, Acc g, Acc gl,
                                         Acc (&S)[StateDim<KIND>::D], Acc& o0, Acc& o1) {
  const bool valid = a.valid.present() ? a.valid.truth(b, t) : true;
  const Acc nt = (a.term.present() && a.term.truth(b, t)) ? Acc(0) : Acc(1);
  if (KIND == 0) {
    const Acc cand = a.r.get<Acc>(b, t) + (g * nt) * S[0];
    if (valid) S[0] = cand;
    o0 = valid ? S[0] : Acc(0);
    o1 = Acc(0);
  } else if (KIND == 1) {
    const Acc V = a.v.get<Acc>(b, t);
    const Acc delta = (a.r.get<Acc>(b, t) + (g * nt) * S[0]) - V;
    const Acc cand = delta + (gl * nt) * S[1];
    const Acc adv = valid ? cand : Acc(0);
    o0 = adv;
    o1 = valid ? adv + V : Acc(0);
    if (valid) { S[0] = V; S[1] = adv; }
  } else {
    const Acc V = a.v.get<Acc>(b, t);
    const Acc delta = (a.r.get<Acc>(b, t) + (g * nt) * a.nv.get<Acc>(b, t)) - V;
    const Acc cand = delta + (gl * nt) * S[0];
    const Acc adv = valid ? cand : Acc(0);
    o0 = adv;
    o1 = valid ? adv + V : Acc(0);
    if (valid) S[0] = adv;
  }
}

template <typename Acc, int KIND>
__global__ __launch_bounds__(SCAN_NT) void reverse_scan_kernel(ScanArgs a) {
  constexpr int D = StateDim<KIND>::D;
  __shared__ Aff<Acc, D> sh_map[SCAN_NT];
  // gamma and gamma*lambda as the reference forms them: python float products
  // rounded to the tensor dtype.
  const Acc g = (Acc)a.gamma;
  const Acc gl = (Acc)(a.gamma * a.lam);
  const int64_t C = (a.T + SCAN_NT - 1) / SCAN_NT;
  for (int64_t b = blockIdx.x; b < a.B; b += gridDim.x) {
    const int64_t t0 = threadIdx.x * C;
    const int64_t t1 = (t0 + C < a.T) ? t0 + C : a.T;
    Aff<Acc, D> f = Aff<Acc, D>::identity();
    for (int64_t t = t1 - 1; t >= t0; --t) f.prepend(step_map<Acc, KIND>(a, b, t, g, gl));
    // Log-depth inclusive suffix scan of the chunk maps (Kogge-Stone over
    // the lanes, through LDS): after the step of distance d, lane j holds
    // P_j = f_j o f_(j+1) o ... o f_(j+2d-1) (the later chunks applied first),
    // and after the last step P_j runs through every chunk from the
    // sequence's end down to chunk j.
    sh_map[threadIdx.x] = f;
    __syncthreads();
    for (int d = 1; d < SCAN_NT; d <<= 1) {
      const bool has = threadIdx.x + d < SCAN_NT;
      Aff<Acc, D> later;
      if (has) later = sh_map[threadIdx.x + d];
      __syncthreads();
      if (has) {
        later.prepend(f);  // `later` first, then this lane's map
        f = later;
      }
      sh_map[threadIdx.x] = f;
      __syncthreads();
    }
    // Chunk j's incoming state: the initial state through P_(j+1).
    Acc S[D];
    if (KIND == 0) S[0] = a.boot.present() ? a.boot.get<Acc>(b, 0) : Acc(0);
    if (KIND == 1) { S[0] = a.boot.present() ? a.boot.get<Acc>(b, 0) : Acc(0); S[1] = Acc(0); }
    if (KIND == 2) S[0] = Acc(0);
    if (threadIdx.x + 1 < SCAN_NT) sh_map[threadIdx.x + 1].apply(S);
    for (int64_t t = t1 - 1; t >= t0; --t) {
      Acc o0, o1;
      ref_step<Acc, KIND>(a, b, t, g, gl, S, o0, o1);
      store_as<Acc>(a.out0, a.odt, b * a.T + t, o0);
      if (KIND != 0) store_as<Acc>(a.out1, a.odt, b * a.T + t, o1);
    }
    __syncthreads();
  }
}

template <int KIND>
int launch_scan(const ScanArgs& a, bool f64, hipStream_t st) {
  if (a.B * a.T == 0) return RRL_OK;
  const unsigned grid = (unsigned)(a.B < 65536 ? a.B : 65536);
  if (f64)
    hipLaunchKernelGGL((reverse_scan_kernel<double, KIND>), dim3(grid), dim3(SCAN_NT), 0, st, a);
  else
    hipLaunchKernelGGL((reverse_scan_kernel<float, KIND>), dim3(grid), dim3(SCAN_NT), 0, st, a);
  return check_launch("reverse_scan_kernel");
}

// ---------------------------------------------------------------------------
// Group statistics: one lane per group (groups are small: G = 4..64 in GRPO).
// ---------------------------------------------------------------------------
template <typename Acc>
__global__ void group_std_kernel(int64_t n, int64_t G, View r, Acc eps, void* out, int odt) {
  for (int64_t gi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; gi < n;
       gi += (int64_t)gridDim.x * blockDim.x) {
    Acc sum = Acc(0);
    Acc lo = r.get<Acc>(gi, 0), hi = lo;
    for (int64_t k = 0; k < G; ++k) {
      const Acc x = r.get<Acc>(gi, k);
      sum += x;
      lo = x < lo ? x : lo;
      hi = x > hi ? x : hi;
    }
    const Acc mean = sum / (Acc)G;
    Acc ss = Acc(0);
    for (int64_t k = 0; k < G; ++k) {
      const Acc d = r.get<Acc>(gi, k) - mean;
      ss += d * d;
    }
    // A uniform group has std 0 exactly ("uniform-reward groups return exactly
    // zero", advantages.py:243-244): the float mean of a non-dyadic value is
    // often an ulp off, which would otherwise leave a std above eps.
    const Acc sd = hi == lo ? Acc(0) : M<Acc>::sqrt(ss / (Acc)G);
    const Acc den = sd > eps ? sd : eps;  // clamp_min(eps) (advantages.py:257)
    for (int64_t k = 0; k < G; ++k) {
      const Acc z = (r.get<Acc>(gi, k) - mean) / den;
      store_as<Acc>(out, odt, gi * G + k, sd > eps ? z : Acc(0));
    }
  }
}

template <typename Acc>
__global__ void leave_one_out_kernel(int64_t n, int64_t G, View r, void* out, int odt) {
  for (int64_t gi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; gi < n;
       gi += (int64_t)gridDim.x * blockDim.x) {
    Acc sum = Acc(0);
    for (int64_t k = 0; k < G; ++k) sum += r.get<Acc>(gi, k);
    for (int64_t k = 0; k < G; ++k) {
      const Acc x = r.get<Acc>(gi, k);
      store_as<Acc>(out, odt, gi * G + k, x - (sum - x) / (Acc)(G - 1));
    }
  }
}

// out[b, t] = mask ? turn_adv[b, id] : 0 (advantages.py:282-290).  The value is
// copied through the accumulation type, which round-trips every float dtype.
template <typename Acc>
__global__ void broadcast_turn_kernel(int64_t B, int64_t K, int64_t T, View adv, View ids,
                                      View mask, void* out, int odt, int32_t* status) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < B * T;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / T, t = i - (i / T) * T;
    const bool m = mask.truth(b, t);
    const int64_t id = load_as<int64_t>(ids.ptr, ids.dt, b * ids.sr + t * ids.sc);
    Acc v = Acc(0);
    if (m) {
      if (id < 0 || id >= K) {
        raise_flag(status, RRL_FLAG_INVALID_TURN);
      } else {
        v = adv.get<Acc>(b, id);
      }
    }
    store_as<Acc>(out, odt, i, v);
  }
}

// ---------------------------------------------------------------------------
// Flat masked reductions over [B, T]: per-block partials, then every consumer
// re-sums the partials in block order (deterministic, no atomics).
// ---------------------------------------------------------------------------
constexpr int RED_NT = 256;
constexpr int RED_MAXB = 1024;

struct RedArgs {
  int64_t B, T;
  View x, mask;
  bool weight;     // mask cast to the value dtype (masked_mean) vs mask != 0
  void* part;      // Acc[RED_MAXB][4]
  double eps;
  int shift;
  void* out;
  int odt;
  int32_t* status;
  const void* grad;
};

inline unsigned red_grid(int64_t n) {
  int64_t g = (n + RED_NT * 8 - 1) / (RED_NT * 8);
  if (g < 1) g = 1;
  if (g > RED_MAXB) g = RED_MAXB;
  return (unsigned)g;
}

template <typename Acc>
__device__ __forceinline__ Acc red_weight(const RedArgs& a, int64_t b, int64_t t) {
  return a.weight ? a.mask.get<Acc>(b, t) : (a.mask.truth(b, t) ? Acc(1) : Acc(0));
}

// Sum of the first two partial columns over all blocks, in block order.
template <typename Acc>
__device__ void sum_partials(const Acc* part, int nb, int col, Acc& out, Acc* sh) {
  Acc v[1] = {Acc(0)};
  for (int i = threadIdx.x; i < nb; i += RED_NT) v[0] += part[i * 4 + col];
  block_sum<RED_NT, 1, Acc>(v, sh);
  out = v[0];
}

// pass 0: part = (sum w*x, sum w); pass 1: part[.,2] = sum w*(x - mean)^2.
template <typename Acc, int PASS>
__global__ __launch_bounds__(RED_NT) void masked_partials_kernel(RedArgs a) {
  __shared__ Acc sh[(RED_NT / 64) * 2];
  Acc* part = static_cast<Acc*>(a.part);
  Acc mean = Acc(0);
  if (PASS == 1) {
    Acc s0, s1;
    sum_partials<Acc>(part, gridDim.x, 0, s0, sh);
    sum_partials<Acc>(part, gridDim.x, 1, s1, sh);
    mean = s0 / s1;
  }
  Acc v[2] = {Acc(0), Acc(0)};
  const int64_t n = a.B * a.T;
  for (int64_t i = blockIdx.x * (int64_t)RED_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * RED_NT) {
    const int64_t b = i / a.T, t = i - (i / a.T) * a.T;
    const Acc w = red_weight<Acc>(a, b, t);
    const Acc x = a.x.get<Acc>(b, t);
    if (PASS == 0) {
      if (a.weight) {
        v[0] += x * w;
        v[1] += w;
      } else if (w != Acc(0)) {
        v[0] += x;
        v[1] += Acc(1);
      }
    } else if (w != Acc(0)) {
      const Acc d = x - mean;
      v[0] += d * d * w;
    }
  }
  block_sum<RED_NT, 2, Acc>(v, sh);
  if (threadIdx.x == 0) {
    if (PASS == 0) {
      part[blockIdx.x * 4 + 0] = v[0];
      part[blockIdx.x * 4 + 1] = v[1];
    } else {
      part[blockIdx.x * 4 + 2] = v[0];
    }
  }
}

// masked_mean finalize: out = sum(w*x) / sum(w).
template <typename Acc>
__global__ __launch_bounds__(RED_NT) void masked_mean_final_kernel(RedArgs a, int nb) {
  __shared__ Acc sh[RED_NT / 64];
  Acc s0, s1;
  sum_partials<Acc>(static_cast<const Acc*>(a.part), nb, 0, s0, sh);
  sum_partials<Acc>(static_cast<const Acc*>(a.part), nb, 1, s1, sh);
  if (threadIdx.x == 0) {
    if (s1 == Acc(0)) raise_flag(a.status, RRL_FLAG_EMPTY_MASK);
    static_cast<Acc*>(a.out)[0] = s0 / s1;
    static_cast<Acc*>(a.part)[RED_MAXB * 4] = s1;  // denominator for the backward
  }
}

template <typename Acc>
__global__ __launch_bounds__(RED_NT) void masked_mean_bwd_kernel(RedArgs a) {
  const Acc G = static_cast<const Acc*>(a.grad)[0];
  const Acc den = static_cast<const Acc*>(a.part)[RED_MAXB * 4];
  const int64_t n = a.B * a.T;
  for (int64_t i = blockIdx.x * (int64_t)RED_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * RED_NT) {
    const int64_t b = i / a.T, t = i - (i / a.T) * a.T;
    static_cast<Acc*>(a.out)[i] = (G / den) * red_weight<Acc>(a, b, t);
  }
}

template <typename Acc>
__global__ __launch_bounds__(RED_NT) void whiten_write_kernel(RedArgs a, int nb) {
  __shared__ Acc sh[RED_NT / 64];
  const Acc* part = static_cast<const Acc*>(a.part);
  Acc s0, s1, s2;
  sum_partials<Acc>(part, nb, 0, s0, sh);
  sum_partials<Acc>(part, nb, 1, s1, sh);
  sum_partials<Acc>(part, nb, 2, s2, sh);
  if (blockIdx.x == 0 && threadIdx.x == 0 && s1 == Acc(0)) raise_flag(a.status, RRL_FLAG_EMPTY_MASK);
  const Acc mean = s0 / s1;
  const Acc sd = M<Acc>::sqrt(s2 / s1);
  const Acc den = sd + (Acc)a.eps;
  const int64_t n = a.B * a.T;
  for (int64_t i = blockIdx.x * (int64_t)RED_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * RED_NT) {
    const int64_t b = i / a.T, t = i - (i / a.T) * a.T;
    const bool m = a.mask.truth(b, t);
    const Acc x = a.x.get<Acc>(b, t);
    const Acc y = a.shift ? (x - mean) / den : x / den;
    store_as<Acc>(a.out, a.odt, i, m ? y : Acc(0));
  }
}

// sequence_log_ratio: one workgroup per row.
template <typename Acc>
__global__ __launch_bounds__(RED_NT) void seq_log_ratio_kernel(int64_t B, int64_t T, View cur,
                                                               View old, View mask, int norm,
                                                               Acc* out, Acc* counts,
                                                               int32_t* status) {
  __shared__ Acc sh[(RED_NT / 64) * 2];
  for (int64_t b = blockIdx.x; b < B; b += gridDim.x) {
    Acc v[2] = {Acc(0), Acc(0)};
    for (int64_t t = threadIdx.x; t < T; t += RED_NT) {
      const Acc w = mask.get<Acc>(b, t);
      v[0] += (cur.get<Acc>(b, t) - old.get<Acc>(b, t)) * w;
      v[1] += w;
    }
    block_sum<RED_NT, 2, Acc>(v, sh);
    if (threadIdx.x == 0) {
      if (v[1] == Acc(0)) raise_flag(status, RRL_FLAG_EMPTY_ROW);
      out[b] = norm ? v[0] / v[1] : v[0];
      counts[b] = v[1];
    }
  }
}

template <typename Acc>
__global__ void seq_log_ratio_bwd_kernel(int64_t B, int64_t T, View mask, int norm,
                                         const Acc* counts, const Acc* grad, Acc* gcur) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < B * T;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / T, t = i - (i / T) * T;
    const Acc w = mask.get<Acc>(b, t);
    gcur[i] = norm ? (grad[b] / counts[b]) * w : grad[b] * w;
  }
}

template <typename Acc>
__global__ void double_sided_kernel(int64_t n, const void* r, int dt, Acc lo, Acc hi, uint8_t* out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const Acc x = load_as<Acc>(r, dt, i);
    out[i] = (x > lo && x < hi) ? 1 : 0;
  }
}

inline unsigned flat_grid(int64_t n, int nt) {
  int64_t g = (n + nt - 1) / nt;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return (unsigned)g;
}

bool view_ok(const rrl_view& v) { return v.ptr == nullptr || is_known_dtype(v.dtype); }

}  // namespace
}  // namespace rrl

using namespace rrl;

static int scan_common(int kind, int64_t B, int64_t T, rrl_view rewards, rrl_view v1, rrl_view v2,
                       rrl_view terminated, rrl_view valid, rrl_view bootstrap, double gamma,
                       double lam, void* out0, void* out1, int32_t out_dtype, void* stream) {
  clear_error();
  RRL_REQUIRE(B >= 0 && T >= 0, RRL_EINVAL, "negative size");
  RRL_REQUIRE(is_float_dtype(out_dtype), RRL_EDTYPE, "output dtype must be floating point");
  RRL_REQUIRE(B * T == 0 || (rewards.ptr && out0), RRL_EINVAL, "null pointer argument");
  RRL_REQUIRE(view_ok(terminated) && view_ok(valid) && view_ok(bootstrap), RRL_EDTYPE,
              "unsupported dtype");
  ScanArgs a{};
  a.B = B; a.T = T;
  a.r = to_view(rewards); a.v = to_view(v1); a.nv = to_view(v2);
  a.term = to_view(terminated); a.valid = to_view(valid); a.boot = to_view(bootstrap);
  a.gamma = gamma; a.lam = lam; a.out0 = out0; a.out1 = out1; a.odt = out_dtype;
  const bool f64 = out_dtype == RRL_F64;
  hipStream_t st = as_stream(stream);
  if (kind == 0) return launch_scan<0>(a, f64, st);
  if (kind == 1) return launch_scan<1>(a, f64, st);
  return launch_scan<2>(a, f64, st);
}

extern "C" int rrl_discounted_returns(int64_t B, int64_t T, rrl_view rewards, rrl_view terminated,
                                      rrl_view valid, rrl_view bootstrap, double gamma, void* out,
                                      int32_t out_dtype, void* stream) {
  rrl_view none{nullptr, RRL_F32, 0, 0};
  return scan_common(0, B, T, rewards, none, none, terminated, valid, bootstrap, gamma, 1.0, out,
                     nullptr, out_dtype, stream);
}

extern "C" int rrl_gae(int64_t B, int64_t T, rrl_view rewards, rrl_view values,
                       rrl_view terminated, rrl_view valid, rrl_view bootstrap, double gamma,
                       double gae_lambda, void* adv_out, void* targets_out, int32_t out_dtype,
                       void* stream) {
  if (B * T != 0 && (!values.ptr || !targets_out)) {
    set_error("values and targets_out are required");
    return RRL_EINVAL;
  }
  rrl_view none{nullptr, RRL_F32, 0, 0};
  return scan_common(1, B, T, rewards, values, none, terminated, valid, bootstrap, gamma,
                     gae_lambda, adv_out, targets_out, out_dtype, stream);
}

extern "C" int rrl_skip_observation_gae(int64_t B, int64_t T, rrl_view rewards,
                                        rrl_view action_end_values, rrl_view next_action_values,
                                        rrl_view terminated, rrl_view valid, double gamma,
                                        double gae_lambda, void* adv_out, void* targets_out,
                                        int32_t out_dtype, void* stream) {
  if (B * T != 0 && (!action_end_values.ptr || !next_action_values.ptr || !targets_out)) {
    set_error("value inputs and targets_out are required");
    return RRL_EINVAL;
  }
  rrl_view none{nullptr, RRL_F32, 0, 0};
  return scan_common(2, B, T, rewards, action_end_values, next_action_values, terminated, valid,
                     none, gamma, gae_lambda, adv_out, targets_out, out_dtype, stream);
}

extern "C" int rrl_group_standardize(int64_t n_groups, int64_t G, rrl_view rewards, double eps,
                                     void* out, int32_t out_dtype, void* stream) {
  clear_error();
  RRL_REQUIRE(n_groups >= 0 && G >= 1, RRL_EINVAL, "bad group shape");
  RRL_REQUIRE(is_float_dtype(out_dtype) && is_float_dtype(rewards.dtype), RRL_EDTYPE,
              "rewards must be floating point");
  if (n_groups == 0) return RRL_OK;
  RRL_REQUIRE(rewards.ptr && out, RRL_EINVAL, "null pointer argument");
  hipStream_t st = as_stream(stream);
  const unsigned grid = flat_grid(n_groups, 256);
  if (out_dtype == RRL_F64)
    hipLaunchKernelGGL((group_std_kernel<double>), dim3(grid), dim3(256), 0, st, n_groups, G,
                       to_view(rewards), (double)eps, out, (int)out_dtype);
  else
    hipLaunchKernelGGL((group_std_kernel<float>), dim3(grid), dim3(256), 0, st, n_groups, G,
                       to_view(rewards), (float)eps, out, (int)out_dtype);
  return check_launch("group_std_kernel");
}

extern "C" int rrl_leave_one_out(int64_t n_groups, int64_t G, rrl_view rewards, void* out,
                                 int32_t out_dtype, void* stream) {
  clear_error();
  RRL_REQUIRE(n_groups >= 0 && G >= 2, RRL_EINVAL, "leave-one-out needs G >= 2");
  RRL_REQUIRE(is_float_dtype(out_dtype) && is_float_dtype(rewards.dtype), RRL_EDTYPE,
              "rewards must be floating point");
  if (n_groups == 0) return RRL_OK;
  RRL_REQUIRE(rewards.ptr && out, RRL_EINVAL, "null pointer argument");
  hipStream_t st = as_stream(stream);
  const unsigned grid = flat_grid(n_groups, 256);
  if (out_dtype == RRL_F64)
    hipLaunchKernelGGL((leave_one_out_kernel<double>), dim3(grid), dim3(256), 0, st, n_groups, G,
                       to_view(rewards), out, (int)out_dtype);
  else
    hipLaunchKernelGGL((leave_one_out_kernel<float>), dim3(grid), dim3(256), 0, st, n_groups, G,
                       to_view(rewards), out, (int)out_dtype);
  return check_launch("leave_one_out_kernel");
}

extern "C" int rrl_broadcast_turn(int64_t B, int64_t K, int64_t T, rrl_view turn_adv,
                                  rrl_view turn_ids, rrl_view mask, void* out, int32_t out_dtype,
                                  int32_t* status, void* stream) {
  clear_error();
  RRL_REQUIRE(B >= 0 && K >= 0 && T >= 0, RRL_EINVAL, "negative size");
  RRL_REQUIRE(is_float_dtype(out_dtype) && is_known_dtype(turn_ids.dtype) &&
                  is_known_dtype(mask.dtype) && is_known_dtype(turn_adv.dtype),
              RRL_EDTYPE, "unsupported dtype");
  if (B * T == 0) return RRL_OK;
  RRL_REQUIRE(turn_ids.ptr && mask.ptr && out && (K == 0 || turn_adv.ptr), RRL_EINVAL,
              "null pointer argument");
  hipStream_t st = as_stream(stream);
  const unsigned grid = flat_grid(B * T, 256);
  if (out_dtype == RRL_F64)
    hipLaunchKernelGGL((broadcast_turn_kernel<double>), dim3(grid), dim3(256), 0, st, B, K, T,
                       to_view(turn_adv), to_view(turn_ids), to_view(mask), out, (int)out_dtype,
                       status);
  else
    hipLaunchKernelGGL((broadcast_turn_kernel<float>), dim3(grid), dim3(256), 0, st, B, K, T,
                       to_view(turn_adv), to_view(turn_ids), to_view(mask), out, (int)out_dtype,
                       status);
  return check_launch("broadcast_turn_kernel");
}

extern "C" size_t rrl_reduce_workspace_bytes(int64_t n) {
  (void)n;
  return (size_t)(RED_MAXB * 4 + 4) * 8 + 256;
}

extern "C" int rrl_masked_mean_fwd(int64_t B, int64_t T, rrl_view values, rrl_view mask,
                                   int32_t acc_dtype, void* workspace, void* out, int32_t* status,
                                   void* stream) {
  clear_error();
  RRL_REQUIRE(B >= 0 && T >= 0, RRL_EINVAL, "negative size");
  RRL_REQUIRE(workspace && out, RRL_EINVAL, "workspace and out are required");
  RRL_REQUIRE(B * T == 0 || (values.ptr && mask.ptr), RRL_EINVAL, "null pointer argument");
  RRL_REQUIRE(is_float_dtype(values.dtype) && is_known_dtype(mask.dtype), RRL_EDTYPE,
              "unsupported dtype");
  RedArgs a{};
  a.B = B; a.T = T; a.x = to_view(values); a.mask = to_view(mask); a.weight = true;
  a.part = workspace; a.out = out; a.status = status;
  const unsigned nb = red_grid(B * T);
  hipStream_t st = as_stream(stream);
  if (acc_dtype == RRL_F64) {
    hipLaunchKernelGGL((masked_partials_kernel<double, 0>), dim3(nb), dim3(RED_NT), 0, st, a);
    if (int rc = check_launch("masked_partials_kernel")) return rc;
    hipLaunchKernelGGL((masked_mean_final_kernel<double>), dim3(1), dim3(RED_NT), 0, st, a, (int)nb);
  } else {
    hipLaunchKernelGGL((masked_partials_kernel<float, 0>), dim3(nb), dim3(RED_NT), 0, st, a);
    if (int rc = check_launch("masked_partials_kernel")) return rc;
    hipLaunchKernelGGL((masked_mean_final_kernel<float>), dim3(1), dim3(RED_NT), 0, st, a, (int)nb);
  }
  return check_launch("masked_mean_final_kernel");
}

extern "C" int rrl_masked_mean_bwd(int64_t B, int64_t T, rrl_view mask, int32_t acc_dtype,
                                   const void* workspace, const void* grad, void* grad_values,
                                   void* stream) {
  clear_error();
  RRL_REQUIRE(workspace && grad && (B * T == 0 || grad_values), RRL_EINVAL, "null pointer argument");
  if (B * T == 0) return RRL_OK;
  RedArgs a{};
  a.B = B; a.T = T; a.mask = to_view(mask); a.weight = true;
  a.part = const_cast<void*>(workspace); a.grad = grad; a.out = grad_values;
  hipStream_t st = as_stream(stream);
  const unsigned grid = flat_grid(B * T, RED_NT);
  if (acc_dtype == RRL_F64)
    hipLaunchKernelGGL((masked_mean_bwd_kernel<double>), dim3(grid), dim3(RED_NT), 0, st, a);
  else
    hipLaunchKernelGGL((masked_mean_bwd_kernel<float>), dim3(grid), dim3(RED_NT), 0, st, a);
  return check_launch("masked_mean_bwd_kernel");
}

extern "C" int rrl_masked_whiten(int64_t B, int64_t T, rrl_view x, rrl_view mask, double eps,
                                 int32_t shift_mean, int32_t acc_dtype, void* workspace, void* out,
                                 int32_t out_dtype, int32_t* status, void* stream) {
  clear_error();
  RRL_REQUIRE(B >= 0 && T >= 0, RRL_EINVAL, "negative size");
  RRL_REQUIRE(workspace && (B * T == 0 || (x.ptr && mask.ptr && out)), RRL_EINVAL,
              "null pointer argument");
  RRL_REQUIRE(is_float_dtype(x.dtype) && is_known_dtype(mask.dtype) && is_float_dtype(out_dtype),
              RRL_EDTYPE, "unsupported dtype");
  RedArgs a{};
  a.B = B; a.T = T; a.x = to_view(x); a.mask = to_view(mask); a.weight = false;
  a.part = workspace; a.eps = eps; a.shift = shift_mean; a.out = out; a.odt = out_dtype;
  a.status = status;
  const unsigned nb = red_grid(B * T);
  hipStream_t st = as_stream(stream);
  if (acc_dtype == RRL_F64) {
    hipLaunchKernelGGL((masked_partials_kernel<double, 0>), dim3(nb), dim3(RED_NT), 0, st, a);
    hipLaunchKernelGGL((masked_partials_kernel<double, 1>), dim3(nb), dim3(RED_NT), 0, st, a);
    hipLaunchKernelGGL((whiten_write_kernel<double>), dim3(nb), dim3(RED_NT), 0, st, a, (int)nb);
  } else {
    hipLaunchKernelGGL((masked_partials_kernel<float, 0>), dim3(nb), dim3(RED_NT), 0, st, a);
    hipLaunchKernelGGL((masked_partials_kernel<float, 1>), dim3(nb), dim3(RED_NT), 0, st, a);
    hipLaunchKernelGGL((whiten_write_kernel<float>), dim3(nb), dim3(RED_NT), 0, st, a, (int)nb);
  }
  return check_launch("masked_whiten");
}

extern "C" int rrl_sequence_log_ratio_fwd(int64_t B, int64_t T, rrl_view cur, rrl_view old,
                                          rrl_view mask, int32_t length_normalize,
                                          int32_t acc_dtype, void* out, void* counts_out,
                                          int32_t* status, void* stream) {
  clear_error();
  RRL_REQUIRE(B >= 0 && T >= 0, RRL_EINVAL, "negative size");
  RRL_REQUIRE(B == 0 || (cur.ptr && old.ptr && mask.ptr && out && counts_out), RRL_EINVAL,
              "null pointer argument");
  RRL_REQUIRE(is_float_dtype(cur.dtype) && is_float_dtype(old.dtype) && is_known_dtype(mask.dtype),
              RRL_EDTYPE, "unsupported dtype");
  if (B == 0) return RRL_OK;
  hipStream_t st = as_stream(stream);
  const unsigned grid = (unsigned)(B < 65536 ? B : 65536);
  if (acc_dtype == RRL_F64)
    hipLaunchKernelGGL((seq_log_ratio_kernel<double>), dim3(grid), dim3(RED_NT), 0, st, B, T,
                       to_view(cur), to_view(old), to_view(mask), (int)length_normalize,
                       static_cast<double*>(out), static_cast<double*>(counts_out), status);
  else
    hipLaunchKernelGGL((seq_log_ratio_kernel<float>), dim3(grid), dim3(RED_NT), 0, st, B, T,
                       to_view(cur), to_view(old), to_view(mask), (int)length_normalize,
                       static_cast<float*>(out), static_cast<float*>(counts_out), status);
  return check_launch("seq_log_ratio_kernel");
}

extern "C" int rrl_sequence_log_ratio_bwd(int64_t B, int64_t T, rrl_view mask,
                                          int32_t length_normalize, int32_t acc_dtype,
                                          const void* counts, const void* grad, void* grad_cur,
                                          void* stream) {
  clear_error();
  RRL_REQUIRE(B * T == 0 || (mask.ptr && counts && grad && grad_cur), RRL_EINVAL,
              "null pointer argument");
  if (B * T == 0) return RRL_OK;
  hipStream_t st = as_stream(stream);
  const unsigned grid = flat_grid(B * T, 256);
  if (acc_dtype == RRL_F64)
    hipLaunchKernelGGL((seq_log_ratio_bwd_kernel<double>), dim3(grid), dim3(256), 0, st, B, T,
                       to_view(mask), (int)length_normalize, static_cast<const double*>(counts),
                       static_cast<const double*>(grad), static_cast<double*>(grad_cur));
  else
    hipLaunchKernelGGL((seq_log_ratio_bwd_kernel<float>), dim3(grid), dim3(256), 0, st, B, T,
                       to_view(mask), (int)length_normalize, static_cast<const float*>(counts),
                       static_cast<const float*>(grad), static_cast<float*>(grad_cur));
  return check_launch("seq_log_ratio_bwd_kernel");
}

extern "C" int rrl_double_sided_mask(int64_t n, const void* ratios, int32_t dtype, double lo,
                                     double hi, uint8_t* out, void* stream) {
  clear_error();
  RRL_REQUIRE(n >= 0, RRL_EINVAL, "negative size");
  RRL_REQUIRE(is_float_dtype(dtype), RRL_EDTYPE, "ratios must be floating point");
  if (n == 0) return RRL_OK;
  RRL_REQUIRE(ratios && out, RRL_EINVAL, "null pointer argument");
  hipStream_t st = as_stream(stream);
  const unsigned grid = flat_grid(n, 256);
  // Thresholds arrive already rounded to the ratio dtype by the caller.
  if (dtype == RRL_F64)
    hipLaunchKernelGGL((double_sided_kernel<double>), dim3(grid), dim3(256), 0, st, n, ratios,
                       (int)dtype, lo, hi, out);
  else
    hipLaunchKernelGGL((double_sided_kernel<float>), dim3(grid), dim3(256), 0, st, n, ratios,
                       (int)dtype, (float)lo, (float)hi, out);
  return check_launch("double_sided_kernel");
}
