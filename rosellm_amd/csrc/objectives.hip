// Policy objectives over [B, T] token log-probs (losses.py:104-512): forward
// scalars and diagnostics, closed-form backward to d/d current_logprobs, and
// the mask denominators for the single-pass kernel.
//
// Work split: one workgroup per sequence row accumulates the row's sums
// (policy_rows_kernel), one workgroup combines rows in a fixed order
// (policy_finalize_kernel).  GSPO-token needs the sequence ratio before its
// token surrogate, so it runs a second row pass.  Every reduction is
// deterministic for a given shape.
#include "policy_math.hpp"
#include "rrl_common.hpp"

namespace rrl {

namespace {

constexpr int RS = 8;  // per-row statistics slots

// Workspace layout (Acc elements): rowstats[B][RS] | seq[B] | globals[8].
template <typename Acc>
struct Workspace {
  Acc* rows;
  Acc* seq;
  Acc* glob;
  __host__ __device__ static Workspace at(void* base, int64_t B) {
    Workspace w;
    w.rows = static_cast<Acc*>(base);
    w.seq = w.rows + B * RS;
    w.glob = w.seq + B;
    return w;
  }
};

struct PolicyArgs {
  rrl_policy_params pp;
  int64_t B, T;
  View cur, old, adv, mask;
  void* ws;
  void* scalars;
  void* seq_out;
  uint8_t* trusted;
  int32_t* status;
  const void* gscal;
  const void* gseq;
  void* grad;
  void* row_coef;
};

// Row pass.  Slots: 0 = #mask-true, 1 = mask weight sum, 2 = sum w*(cur-old),
// 3..6 = objective-specific sums (see policy_finalize_kernel).
template <typename Acc, int NT, bool STATS_ONLY>
__global__ __launch_bounds__(NT) void policy_rows_kernel(PolicyArgs a) {
  __shared__ Acc sh[(NT / 64) * 7];
  const PolicyConsts<Acc> c = PolicyConsts<Acc>::make(a.pp);
  Workspace<Acc> ws = Workspace<Acc>::at(a.ws, a.B);
  for (int64_t b = blockIdx.x; b < a.B; b += gridDim.x) {
    Acc v[7] = {Acc(0), Acc(0), Acc(0), Acc(0), Acc(0), Acc(0), Acc(0)};
    for (int64_t t = threadIdx.x; t < a.T; t += NT) {
      const Acc w = mask_weight<Acc>(c, a.mask, b, t);
      const bool mt = c.kind == RRL_OBJ_NLL ? w != Acc(0) : a.mask.truth(b, t);
      v[0] += mt ? Acc(1) : Acc(0);
      v[1] += w;
      if (STATS_ONLY) continue;
      const Acc l = a.cur.get<Acc>(b, t);
      const Acc o = a.old.get<Acc>(b, t);
      if (c.kind == RRL_OBJ_NLL) {
        // An ignored token's log-prob may be NaN (no target): select, not multiply.
        v[3] += w != Acc(0) ? l * w : Acc(0);
        continue;
      }
      v[2] += (l - o) * w;
      if (c.kind == RRL_OBJ_PPO) {
        const Acc A = a.adv.get<Acc>(b, t);
        Acc rho, safe, d;
        const Acc surr = ppo_token(c, l, o, A, rho, safe, d);
        v[3] += surr * w;
        v[4] += ((rho - Acc(1)) - safe) * w;
        v[5] += ((rho < c.lo) || (rho > c.hi) ? Acc(1) : Acc(0)) * w;
        v[6] += rho * w;
      } else if (c.kind == RRL_OBJ_SAO) {
        const Acc A = a.adv.get<Acc>(b, t);
        Acc rho, safe, d, drho;
        bool tr;
        const Acc term = sao_token(c, l, o, A, rho, safe, tr, d, drho);
        v[3] += term * w;
        v[4] += ((rho - Acc(1)) - safe) * w;
        v[5] += (tr ? Acc(0) : Acc(1)) * w;
        v[6] += rho * w;
        if (a.trusted) a.trusted[b * a.T + t] = (tr && mt) ? 1 : 0;
      } else if (c.kind == RRL_OBJ_SAPO) {
        const Acc A = a.adv.get<Acc>(b, t);
        Acc rho, safe, p, d, dp;
        const Acc soft = sapo_token(c, l, o, A, rho, safe, p, d, dp);
        v[3] += soft * w;
        v[4] += ((rho - Acc(1)) - safe) * w;
        v[5] += rho * w;
        v[6] += ((Acc(4) * p) * (Acc(1) - p)) * w;
      }
    }
    block_sum<NT, 7, Acc>(v, sh);
    if (threadIdx.x == 0) {
#pragma unroll
      for (int k = 0; k < 7; ++k) ws.rows[b * RS + k] = v[k];
    }
  }
}

// GSPO sequence ratio from row sums (losses.py:252-256): returns s, writes the
// clamped log ratio and whether the clamp passed gradient.
template <typename Acc>
__device__ __forceinline__ Acc gspo_seq_ratio(const PolicyConsts<Acc>& c, Acc lr, Acc cnt,
                                              Acc& safe, Acc& pass) {
  const Acc y = lr / cnt;
  safe = clampt(y, -c.K, c.K);
  pass = clamp_pass(y, -c.K, c.K);
  return M<Acc>::exp(safe);
}

// d min(s*A, clamp(s, lo, hi)*A) / d s with torch.minimum's tie split.
template <typename Acc>
__device__ __forceinline__ Acc clipped_surrogate(const PolicyConsts<Acc>& c, Acc s, Acc A,
                                                 Acc& dsurr) {
  const Acc cs = clampt(s, c.lo, c.hi);
  Acc share;
  const Acc surr = min_with_share(s * A, cs * A, share);
  dsurr = share * A + (Acc(1) - share) * A * clamp_pass(s, c.lo, c.hi);
  return surr;
}

template <typename Acc, int NT>
__global__ __launch_bounds__(NT) void policy_finalize_kernel(PolicyArgs a) {
  __shared__ Acc sh[(NT / 64) * 8];
  const PolicyConsts<Acc> c = PolicyConsts<Acc>::make(a.pp);
  Workspace<Acc> ws = Workspace<Acc>::at(a.ws, a.B);
  Acc v[8] = {Acc(0), Acc(0), Acc(0), Acc(0), Acc(0), Acc(0), Acc(0), Acc(0)};
  const bool per_seq = c.kind == RRL_OBJ_GSPO || c.kind == RRL_OBJ_GSPO_TOKEN || c.kind == RRL_OBJ_SAPO;
  for (int64_t b = threadIdx.x; b < a.B; b += NT) {
    const Acc* rs = ws.rows + b * RS;
    const Acc cnt = rs[0];
    if (per_seq) v[7] += (cnt == Acc(0)) ? Acc(1) : Acc(0);
    if (c.kind == RRL_OBJ_PPO || c.kind == RRL_OBJ_SAO || c.kind == RRL_OBJ_NLL) {
      v[0] += rs[1];
      v[3] += rs[3];
      v[4] += rs[4];
      v[5] += rs[5];
      v[6] += rs[6];
    } else if (c.kind == RRL_OBJ_GSPO || c.kind == RRL_OBJ_GSPO_TOKEN) {
      Acc safe, pass, dsurr;
      const Acc s = gspo_seq_ratio(c, rs[2], cnt, safe, pass);
      ws.seq[b] = s;
      if (a.seq_out) store_as<Acc>(a.seq_out, sizeof(Acc) == 8 ? RRL_F64 : RRL_F32, b, s);
      if (c.kind == RRL_OBJ_GSPO) {
        const Acc A = a.adv.get<Acc>(b, 0);
        v[3] += clipped_surrogate(c, s, A, dsurr);
      }
      v[4] += (s - Acc(1)) - safe;
      v[5] += ((s < c.lo) || (s > c.hi)) ? Acc(1) : Acc(0);
      v[6] += s;
    } else {  // SAPO: per-sequence means, then mean over sequences
      v[3] += rs[3] / cnt;
      v[4] += rs[4] / cnt;
      v[5] += rs[5] / cnt;
      v[6] += rs[6] / cnt;
    }
  }
  block_sum<NT, 8, Acc>(v, sh);
  if (threadIdx.x == 0) {
    Acc* out = static_cast<Acc*>(a.scalars);
    for (int k = 0; k < RRL_NSCALARS; ++k) out[k] = Acc(0);
    if (c.kind == RRL_OBJ_NLL) {
      // F.cross_entropy: "mean" divides by the number of non-ignored tokens
      // (NaN when there is none, no error); "sum" does not divide.
      const bool sum = (a.pp.flags & RRL_POLICY_SUM) != 0;
      ws.glob[0] = sum ? Acc(1) : v[0];
      out[0] = sum ? v[3] : v[3] / v[0];
      out[1] = v[0];
    } else if (c.kind == RRL_OBJ_PPO || c.kind == RRL_OBJ_SAO) {
      const Acc Mw = v[0];
      if (Mw == Acc(0)) raise_flag(a.status, RRL_FLAG_EMPTY_MASK);
      ws.glob[0] = Mw;
      out[0] = v[3] / Mw;
      out[1] = v[4] / Mw;
      out[2] = v[5] / Mw;
      out[3] = v[6] / Mw;
    } else {
      if (v[7] != Acc(0)) raise_flag(a.status, RRL_FLAG_EMPTY_ROW);
      const Acc Bf = (Acc)a.B;
      ws.glob[0] = Bf;
      if (c.kind == RRL_OBJ_SAPO) {
        out[0] = v[3] / Bf;
        out[1] = v[4] / Bf;
        out[2] = v[5] / Bf;
        out[3] = v[6] / Bf;
      } else {
        out[0] = v[3] / Bf;  // GSPO-token overwrites after its second pass
        out[1] = v[4] / Bf;
        out[2] = v[5] / Bf;
        out[3] = v[6] / Bf;
      }
    }
  }
}

// GSPO-token second pass: per-row sum of mask * min(tau*A, clip(tau)*A) with
// tau = sg(s) * exp(cur - sg(cur)) (losses.py:331-341).
template <typename Acc, int NT>
__global__ __launch_bounds__(NT) void gspo_token_rows_kernel(PolicyArgs a) {
  __shared__ Acc sh[NT / 64];
  const PolicyConsts<Acc> c = PolicyConsts<Acc>::make(a.pp);
  Workspace<Acc> ws = Workspace<Acc>::at(a.ws, a.B);
  for (int64_t b = blockIdx.x; b < a.B; b += gridDim.x) {
    const Acc s = ws.seq[b];
    Acc v[1] = {Acc(0)};
    for (int64_t t = threadIdx.x; t < a.T; t += NT) {
      const Acc w = mask_weight<Acc>(c, a.mask, b, t);
      const Acc l = a.cur.get<Acc>(b, t);
      const Acc tau = s * M<Acc>::exp(l - l);
      Acc d;
      v[0] += clipped_surrogate(c, tau, a.adv.get<Acc>(b, t), d) * w;
    }
    block_sum<NT, 1, Acc>(v, sh);
    if (threadIdx.x == 0) ws.rows[b * RS + 3] = v[0];
  }
}

template <typename Acc, int NT>
__global__ __launch_bounds__(NT) void gspo_token_finalize_kernel(PolicyArgs a) {
  __shared__ Acc sh[NT / 64];
  Workspace<Acc> ws = Workspace<Acc>::at(a.ws, a.B);
  Acc v[1] = {Acc(0)};
  for (int64_t b = threadIdx.x; b < a.B; b += NT) v[0] += ws.rows[b * RS + 3] / ws.rows[b * RS + 0];
  block_sum<NT, 1, Acc>(v, sh);
  if (threadIdx.x == 0) static_cast<Acc*>(a.scalars)[0] = v[0] / (Acc)a.B;
}

// Backward: grad_cur[b, t] = sum_k G[k] d scalar_k / d cur[b, t].
template <typename Acc, int NT>
__global__ __launch_bounds__(NT) void policy_bwd_kernel(PolicyArgs a) {
  const PolicyConsts<Acc> c = PolicyConsts<Acc>::make(a.pp);
  Workspace<Acc> ws = Workspace<Acc>::at(a.ws, a.B);
  const Acc* G = static_cast<const Acc*>(a.gscal);
  const Acc G0 = G[0], G1 = G[1], G2 = G[2], G3 = G[3];
  Acc* grad = static_cast<Acc*>(a.grad);
  const Acc Bf = (Acc)a.B;
  for (int64_t b = blockIdx.x; b < a.B; b += gridDim.x) {
    const Acc* rs = ws.rows + b * RS;
    const Acc cnt = rs[0];
    // Per-row factor for the GSPO kinds' sequence-ratio terms.
    Acc seq_coef = Acc(0), s = Acc(0);
    if (c.kind == RRL_OBJ_GSPO || c.kind == RRL_OBJ_GSPO_TOKEN) {
      Acc safe, pass, dsurr = Acc(0);
      s = gspo_seq_ratio(c, rs[2], cnt, safe, pass);
      const Acc gs = a.gseq ? static_cast<const Acc*>(a.gseq)[b] : Acc(0);
      Acc dy = (G1 * (s - Acc(1)) + G3 * s) / Bf + gs * s;
      if (c.kind == RRL_OBJ_GSPO) {
        (void)clipped_surrogate(c, s, a.adv.get<Acc>(b, 0), dsurr);
        dy += (G0 * dsurr * s) / Bf;
      }
      seq_coef = dy * pass;
    }
    for (int64_t t = threadIdx.x; t < a.T; t += NT) {
      const Acc w = mask_weight<Acc>(c, a.mask, b, t);
      Acc gr = Acc(0);
      if (c.kind == RRL_OBJ_NLL) {
        gr = w != Acc(0) ? (w / ws.glob[0]) * G0 : Acc(0);
      } else if (c.kind == RRL_OBJ_PPO) {
        const Acc l = a.cur.get<Acc>(b, t), o = a.old.get<Acc>(b, t), A = a.adv.get<Acc>(b, t);
        Acc rho, safe, d;
        (void)ppo_token(c, l, o, A, rho, safe, d);
        const Acc px = clamp_pass(l - o, -c.K, c.K);
        const Acc drho = rho * px;
        gr = (w / ws.glob[0]) * (G0 * d + G1 * (drho - px) + G3 * drho);
      } else if (c.kind == RRL_OBJ_SAO) {
        const Acc l = a.cur.get<Acc>(b, t), o = a.old.get<Acc>(b, t), A = a.adv.get<Acc>(b, t);
        Acc rho, safe, d, drho;
        bool tr;
        (void)sao_token(c, l, o, A, rho, safe, tr, d, drho);
        const Acc px = clamp_pass(l - o, -c.K, c.K);
        gr = (w / ws.glob[0]) * (G0 * d + G1 * (drho - px) + G3 * drho);
      } else if (c.kind == RRL_OBJ_SAPO) {
        const Acc l = a.cur.get<Acc>(b, t), o = a.old.get<Acc>(b, t), A = a.adv.get<Acc>(b, t);
        Acc rho, safe, p, d, dp;
        (void)sapo_token(c, l, o, A, rho, safe, p, d, dp);
        const Acc px = clamp_pass(l - o, -c.K, c.K);
        const Acc drho = rho * px;
        const Acc dgate = (Acc(4) * dp) * (Acc(1) - Acc(2) * p);
        gr = ((w / cnt) / Bf) * (G0 * d + G1 * (drho - px) + G2 * drho + G3 * dgate);
      } else if (c.kind == RRL_OBJ_GSPO) {
        gr = seq_coef * (w / cnt);
      } else {  // GSPO-token
        const Acc l = a.cur.get<Acc>(b, t);
        const Acc tau = s * M<Acc>::exp(l - l);
        Acc d;
        (void)clipped_surrogate(c, tau, a.adv.get<Acc>(b, t), d);
        gr = ((w / cnt) / Bf) * (G0 * d * tau) + seq_coef * (w / cnt);
      }
      grad[b * a.T + t] = gr;
    }
  }
}

// Mask denominators for the single-pass kernel.
template <typename Acc, int NT>
__global__ __launch_bounds__(NT) void row_coef_kernel(PolicyArgs a) {
  __shared__ Acc sh[(NT / 64) * 2];
  Workspace<Acc> ws = Workspace<Acc>::at(a.ws, a.B);
  Acc v[2] = {Acc(0), Acc(0)};
  for (int64_t b = threadIdx.x; b < a.B; b += NT) {
    v[0] += ws.rows[b * RS + 1];
    v[1] += (ws.rows[b * RS + 0] == Acc(0)) ? Acc(1) : Acc(0);
  }
  block_sum<NT, 2, Acc>(v, sh);
  const bool per_seq = a.pp.kind == RRL_OBJ_SAPO;
  const bool nll = a.pp.kind == RRL_OBJ_NLL;
  if (threadIdx.x == 0) {
    if (!per_seq && !nll && v[0] == Acc(0)) raise_flag(a.status, RRL_FLAG_EMPTY_MASK);
    if (per_seq && v[1] != Acc(0)) raise_flag(a.status, RRL_FLAG_EMPTY_ROW);
  }
  Acc* coef = static_cast<Acc*>(a.row_coef);
  const Acc Bf = (Acc)a.B;
  const Acc flat = (nll && (a.pp.flags & RRL_POLICY_SUM)) ? Acc(1) : Acc(1) / v[0];
  for (int64_t b = threadIdx.x; b < a.B; b += NT) {
    coef[b] = per_seq ? (Acc(1) / ws.rows[b * RS + 0]) / Bf : flat;
  }
}

template <typename Acc>
int run_policy_fwd(const PolicyArgs& a, hipStream_t st) {
  constexpr int NT = 256;
  const unsigned grid = (unsigned)(a.B < 65536 ? a.B : 65536);
  if (a.B > 0) {
    hipLaunchKernelGGL((policy_rows_kernel<Acc, NT, false>), dim3(grid), dim3(NT), 0, st, a);
    if (int rc = check_launch("policy_rows_kernel")) return rc;
  }
  hipLaunchKernelGGL((policy_finalize_kernel<Acc, 1024>), dim3(1), dim3(1024), 0, st, a);
  if (int rc = check_launch("policy_finalize_kernel")) return rc;
  if (a.pp.kind == RRL_OBJ_GSPO_TOKEN && a.B > 0) {
    hipLaunchKernelGGL((gspo_token_rows_kernel<Acc, NT>), dim3(grid), dim3(NT), 0, st, a);
    if (int rc = check_launch("gspo_token_rows_kernel")) return rc;
    hipLaunchKernelGGL((gspo_token_finalize_kernel<Acc, 1024>), dim3(1), dim3(1024), 0, st, a);
    if (int rc = check_launch("gspo_token_finalize_kernel")) return rc;
  }
  return RRL_OK;
}

// Target ids in [0, V) (NLL's ignore_index exempt), one token per thread,
// ahead of the single-pass sweep that makes the same check.
struct TargetCheckArgs {
  rrl_policy_params pp;
  int64_t B, T, V;
  View tgt;
  int32_t* status;
};

__global__ __launch_bounds__(256) void check_targets_kernel(TargetCheckArgs a) {
  const PolicyConsts<float> c = PolicyConsts<float>::make(a.pp);
  const int64_t n = a.B * a.T;
  bool bad = false;
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t b = i / a.T, t = i - b * a.T;
    const int64_t tgt = load_index(a.tgt.ptr, a.tgt.dt, b * a.tgt.sr + t * a.tgt.sc);
    bad = bad || ((tgt < 0 || tgt >= a.V) && !target_ignored(c, tgt));
  }
  if (__any(bad) && (threadIdx.x & 63) == 0) raise_flag(a.status, RRL_FLAG_TARGET_RANGE);
}

int validate_policy(const rrl_policy_params* p, int64_t B, int64_t T, int acc) {
  RRL_REQUIRE(p != nullptr, RRL_EINVAL, "params is null");
  RRL_REQUIRE(p->kind >= RRL_OBJ_PPO && p->kind <= RRL_OBJ_NLL, RRL_EINVAL, "unknown objective kind");
  RRL_REQUIRE(B >= 0 && T >= 0, RRL_EINVAL, "negative size");
  RRL_REQUIRE(acc == RRL_F32 || acc == RRL_F64, RRL_EDTYPE, "acc dtype must be float32 or float64");
  return RRL_OK;
}

}  // namespace
}  // namespace rrl

using namespace rrl;

extern "C" size_t rrl_policy_workspace_bytes(int64_t B, int32_t acc_dtype) {
  const size_t e = acc_dtype == RRL_F64 ? 8 : 4;
  return (size_t)(B * RS + B + 8) * e + 256;
}

extern "C" int rrl_policy_fwd(const rrl_policy_params* params, int64_t B, int64_t T,
                              rrl_view cur, rrl_view old, rrl_view adv, rrl_view mask,
                              int32_t acc_dtype, void* workspace, void* scalars_out,
                              void* seq_out, uint8_t* trusted_out, int32_t* status,
                              void* stream) {
  clear_error();
  if (int rc = validate_policy(params, B, T, acc_dtype)) return rc;
  RRL_REQUIRE(workspace && scalars_out, RRL_EINVAL, "workspace and scalars_out are required");
  RRL_REQUIRE(B * T == 0 || (cur.ptr && old.ptr && adv.ptr && mask.ptr), RRL_EINVAL,
              "null input pointer");
  RRL_REQUIRE(is_float_dtype(cur.dtype) && is_float_dtype(old.dtype) && is_float_dtype(adv.dtype),
              RRL_EDTYPE, "log-probabilities and advantages must be floating point");
  RRL_REQUIRE(is_known_dtype(mask.dtype), RRL_EDTYPE, "unsupported mask dtype");
  RRL_REQUIRE(params->kind != RRL_OBJ_NLL || mask.dtype == RRL_I32 || mask.dtype == RRL_I64,
              RRL_EDTYPE, "NLL: the mask operand holds the target ids (int32 or int64)");
  PolicyArgs a{};
  a.pp = *params; a.B = B; a.T = T;
  a.cur = to_view(cur); a.old = to_view(old); a.adv = to_view(adv); a.mask = to_view(mask);
  a.ws = workspace; a.scalars = scalars_out; a.seq_out = seq_out; a.trusted = trusted_out;
  a.status = status;
  hipStream_t st = as_stream(stream);
  return acc_dtype == RRL_F64 ? run_policy_fwd<double>(a, st) : run_policy_fwd<float>(a, st);
}

extern "C" int rrl_policy_bwd(const rrl_policy_params* params, int64_t B, int64_t T,
                              rrl_view cur, rrl_view old, rrl_view adv, rrl_view mask,
                              int32_t acc_dtype, const void* workspace, const void* grad_scalars,
                              const void* grad_seq, void* grad_cur, void* stream) {
  clear_error();
  if (int rc = validate_policy(params, B, T, acc_dtype)) return rc;
  RRL_REQUIRE(workspace && grad_scalars && (B * T == 0 || grad_cur), RRL_EINVAL,
              "workspace, grad_scalars and grad_cur are required");
  if (B * T == 0) return RRL_OK;
  PolicyArgs a{};
  a.pp = *params; a.B = B; a.T = T;
  a.cur = to_view(cur); a.old = to_view(old); a.adv = to_view(adv); a.mask = to_view(mask);
  a.ws = const_cast<void*>(workspace); a.gscal = grad_scalars; a.gseq = grad_seq; a.grad = grad_cur;
  constexpr int NT = 256;
  const unsigned grid = (unsigned)(B < 65536 ? B : 65536);
  hipStream_t st = as_stream(stream);
  if (acc_dtype == RRL_F64)
    hipLaunchKernelGGL((policy_bwd_kernel<double, NT>), dim3(grid), dim3(NT), 0, st, a);
  else
    hipLaunchKernelGGL((policy_bwd_kernel<float, NT>), dim3(grid), dim3(NT), 0, st, a);
  return check_launch("policy_bwd_kernel");
}

extern "C" int rrl_policy_row_coef(const rrl_policy_params* params, int64_t B, int64_t T,
                                   rrl_view mask, int32_t acc_dtype, void* row_coef,
                                   void* workspace, int32_t* status, void* stream) {
  clear_error();
  if (int rc = validate_policy(params, B, T, acc_dtype)) return rc;
  RRL_REQUIRE(params->kind == RRL_OBJ_PPO || params->kind == RRL_OBJ_SAO ||
                  params->kind == RRL_OBJ_SAPO || params->kind == RRL_OBJ_NLL,
              RRL_EINVAL, "row coefficients exist for the token-local objectives only");
  RRL_REQUIRE(workspace && (B == 0 || (row_coef && mask.ptr)), RRL_EINVAL, "null pointer argument");
  RRL_REQUIRE(is_known_dtype(mask.dtype), RRL_EDTYPE, "unsupported mask dtype");
  RRL_REQUIRE(params->kind != RRL_OBJ_NLL || mask.dtype == RRL_I32 || mask.dtype == RRL_I64,
              RRL_EDTYPE, "NLL: the mask operand holds the target ids (int32 or int64)");
  PolicyArgs a{};
  a.pp = *params; a.B = B; a.T = T; a.mask = to_view(mask);
  a.ws = workspace; a.row_coef = row_coef; a.status = status;
  constexpr int NT = 256;
  const unsigned grid = (unsigned)(B < 65536 ? B : 65536);
  hipStream_t st = as_stream(stream);
  if (B > 0) {
    if (acc_dtype == RRL_F64)
      hipLaunchKernelGGL((policy_rows_kernel<double, NT, true>), dim3(grid), dim3(NT), 0, st, a);
    else
      hipLaunchKernelGGL((policy_rows_kernel<float, NT, true>), dim3(grid), dim3(NT), 0, st, a);
    if (int rc = check_launch("policy_rows_kernel(stats)")) return rc;
  }
  if (acc_dtype == RRL_F64)
    hipLaunchKernelGGL((row_coef_kernel<double, 1024>), dim3(1), dim3(1024), 0, st, a);
  else
    hipLaunchKernelGGL((row_coef_kernel<float, 1024>), dim3(1), dim3(1024), 0, st, a);
  return check_launch("row_coef_kernel");
}

extern "C" int rrl_check_targets(const rrl_policy_params* params, int64_t B, int64_t T,
                                 int64_t V, rrl_view target, int32_t* status, void* stream) {
  clear_error();
  if (int rc = validate_policy(params, B, T, RRL_F32)) return rc;
  RRL_REQUIRE(V >= 1, RRL_EINVAL, "vocabulary must be non-empty");
  RRL_REQUIRE(status && (B * T == 0 || target.ptr), RRL_EINVAL, "null pointer argument");
  RRL_REQUIRE(target.dtype == RRL_I32 || target.dtype == RRL_I64, RRL_EDTYPE,
              "target ids must be int32 or int64");
  const int64_t n = B * T;
  if (n == 0) return RRL_OK;
  TargetCheckArgs a{};
  a.pp = *params; a.B = B; a.T = T; a.V = V; a.tgt = to_view(target); a.status = status;
  const int64_t blocks = (n + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 4096 ? blocks : 4096);
  hipLaunchKernelGGL(check_targets_kernel, dim3(grid), dim3(256), 0, as_stream(stream), a);
  return check_launch("check_targets_kernel");
}
