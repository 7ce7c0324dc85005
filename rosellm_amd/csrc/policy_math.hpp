// Per-token objective terms and their derivatives with respect to the current
// log-prob, written as the same op sequence the reference evaluates so that
// threshold decisions (clamp bounds, minimum ties, strict trust bounds) match.
#pragma once

#include "rrl_common.hpp"

namespace rrl {

template <typename Acc>
struct PolicyConsts {
  Acc lo, hi;        // acc(1 - clip_low), acc(1 + clip_high)
  Acc K;             // max_log_ratio
  Acc tau_pos, tau_neg;
  bool detach;
  int kind;
  bool mask_is_weight;
  int64_t ignore_index;  // NLL only
  __host__ __device__ static PolicyConsts make(const rrl_policy_params& p) {
    PolicyConsts c;
    c.lo = (Acc)(1.0 - p.clip_low);
    c.hi = (Acc)(1.0 + p.clip_high);
    c.K = (Acc)p.max_log_ratio;
    c.tau_pos = (Acc)p.tau_positive;
    c.tau_neg = (Acc)p.tau_negative;
    c.detach = p.detach_ratio != 0;
    c.kind = p.kind;
    c.mask_is_weight = p.mask_is_weight != 0;
    c.ignore_index = p.ignore_index;
    return c;
  }
};

// PPO/GRPO token surrogate min(rho*A, clip(rho)*A) (losses.py:462-470) and
// d surrogate / d logp, following autograd through clamp -> exp -> clamp ->
// minimum.
template <typename Acc>
__device__ __forceinline__ Acc ppo_token(const PolicyConsts<Acc>& c, Acc l, Acc lo_old, Acc A,
                                         Acc& rho, Acc& safe, Acc& dsurr) {
  const Acc x = l - lo_old;
  safe = clampt(x, -c.K, c.K);
  rho = M<Acc>::exp(safe);
  const Acc cr = clampt(rho, c.lo, c.hi);
  const Acc u = rho * A;
  const Acc v = cr * A;
  Acc share;
  const Acc surr = min_with_share(u, v, share);
  const Acc grad_rho = share * A + (Acc(1) - share) * A * clamp_pass(rho, c.lo, c.hi);
  dsurr = grad_rho * rho * clamp_pass(x, -c.K, c.K);
  return surr;
}

// SAO/DIS term where(trusted, iw*A*logp, 0) (losses.py:178-190) and its derivative.
template <typename Acc>
__device__ __forceinline__ Acc sao_token(const PolicyConsts<Acc>& c, Acc l, Acc lo_roll, Acc A,
                                         Acc& rho, Acc& safe, bool& trusted, Acc& dterm,
                                         Acc& drho_dl) {
  const Acc x = l - lo_roll;
  safe = clampt(x, -c.K, c.K);
  rho = M<Acc>::exp(safe);
  trusted = (rho > c.lo) && (rho < c.hi);
  drho_dl = rho * clamp_pass(x, -c.K, c.K);
  Acc term = Acc(0);
  dterm = Acc(0);
  if (trusted) {
    const Acc ia = rho * A;
    term = ia * l;
    dterm = ia;
    if (!c.detach) dterm += (l * A) * drho_dl;
  }
  return term;
}

// SAPO soft surrogate (4/tau)*sigmoid(tau*(rho-1))*A (losses.py:399-412).
// Returns the surrogate; p is the sigmoid, dsoft = d surrogate / d logp,
// dp = d p / d logp.
template <typename Acc>
__device__ __forceinline__ Acc sapo_token(const PolicyConsts<Acc>& c, Acc l, Acc lo_roll, Acc A,
                                          Acc& rho, Acc& safe, Acc& p, Acc& dsoft, Acc& dp) {
  const Acc x = l - lo_roll;
  safe = clampt(x, -c.K, c.K);
  rho = M<Acc>::exp(safe);
  const Acc tau = A > Acc(0) ? c.tau_pos : c.tau_neg;
  const Acc z = tau * (rho - Acc(1));
  p = Acc(1) / (Acc(1) + M<Acc>::exp(-z));
  const Acc soft = ((Acc(4) / tau) * p) * A;
  dp = (p * (Acc(1) - p)) * tau * rho * clamp_pass(x, -c.K, c.K);
  dsoft = ((Acc(4) / tau) * A) * dp;
  return soft;
}

// d(token term)/d logp used by the single-pass kernel for the token-local
// objectives (PPO, SAO, SAPO, and NLL, whose term is logp itself).
template <typename Acc>
__device__ __forceinline__ Acc token_local_grad(const PolicyConsts<Acc>& c, Acc l, Acc o, Acc A) {
  if (c.kind == RRL_OBJ_NLL) return Acc(1);
  Acc rho, safe;
  if (c.kind == RRL_OBJ_PPO) {
    Acc d;
    (void)ppo_token(c, l, o, A, rho, safe, d);
    return d;
  }
  if (c.kind == RRL_OBJ_SAO) {
    bool tr;
    Acc d, drho;
    (void)sao_token(c, l, o, A, rho, safe, tr, d, drho);
    return d;
  }
  Acc p, d, dp;
  (void)sapo_token(c, l, o, A, rho, safe, p, d, dp);
  return d;
}

// Weight of token (b, t) in the objective's sum (mask semantics per function).
// For NLL the mask operand holds the target ids: weight 1 unless the id is
// F.cross_entropy's ignore_index.
template <typename Acc>
__device__ __forceinline__ Acc mask_weight(const PolicyConsts<Acc>& c, const View& mask,
                                           int64_t b, int64_t t) {
  if (c.kind == RRL_OBJ_NLL)
    return load_index(mask.ptr, mask.dt, b * mask.sr + t * mask.sc) != c.ignore_index ? Acc(1)
                                                                                     : Acc(0);
  return c.mask_is_weight ? mask.get<Acc>(b, t) : (mask.truth(b, t) ? Acc(1) : Acc(0));
}

// Whether target id `tgt` is exempt from the [0, V) range check: NLL's ignored
// ids, which carry no loss (F.cross_entropy skips them).
template <typename Acc>
__device__ __forceinline__ bool target_ignored(const PolicyConsts<Acc>& c, int64_t tgt) {
  return c.kind == RRL_OBJ_NLL && tgt == c.ignore_index;
}

// Mask weight times the row coefficient, exactly 0 for a zero weight even when
// the coefficient is infinite (NLL's "mean" over an all-ignored batch, 1/0).
template <typename Acc>
__device__ __forceinline__ Acc weight_coef(Acc w, Acc coef) {
  return w == Acc(0) ? Acc(0) : w * coef;
}

}  // namespace rrl
