// Token log-probs over the vocabulary (losses.py:14-38), their backward, and the
// single-pass log-prob + token-local objective gradient.
//
// One workgroup owns one logits row (b, t).  Sweep 1 streams the row with
// 16-byte loads and keeps an online (max, sum exp) pair per lane, combined
// across the wave with shuffles and across waves through LDS.  Sweep 2 (backward
// and single pass) writes dlogits = g * (onehot - exp(x - lse)), so no softmax
// tensor is ever materialised.  The register-resident kernels
// (logprob_resident.hip) keep the whole row in registers between the sweeps for
// bf16, f16 and float32 rows up to 163840 (16-bit) or 81920 (float32) entries;
// this file is the generic path for float64, longer rows, accumulation and
// dlogits rows laid out differently from the logits rows.
#include <mutex>

#include "policy_math.hpp"
#include "rrl_common.hpp"
#include "row_common.hpp"

namespace rrl {

namespace {

enum Mode { MODE_FWD = 0, MODE_BWD = 1, MODE_FUSED = 2 };

template <class Tag, int MODE, int NT>
__global__ __launch_bounds__(NT) void row_kernel(RowArgs a) {
  using S = typename Tag::S;
  using Acc = typename Tag::Acc;
  constexpr int VEC = Tag::VEC;
  __shared__ Acc sh_m[NT / 64];
  __shared__ Acc sh_s[NT / 64];

  const int64_t rows = a.B * a.T;
  // A conditional rerun (RRL_POLICY_RERUN_FAST_RANGE) does the call again
  // only when the register-resident launch before it flagged a row outside
  // its exponent range; otherwise every workgroup returns here.
  if (MODE == MODE_FUSED && (a.pp.flags & RRL_POLICY_RERUN_FAST_RANGE) &&
      (*static_cast<const volatile int32_t*>(a.status) & RRL_FLAG_FAST_RANGE) == 0)
    return;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int64_t b = r / a.T, t = r - (r / a.T) * a.T;
    const S* row = static_cast<const S*>(a.logits) + b * a.ls_b + t * a.ls_t;
    const RowSplit sp = RowSplit::make<S, VEC>(row, a.V);
    // The target id and logit are uniform over the workgroup.
    const int64_t tgt = load_index(a.tgt.ptr, a.tgt.dt, b * a.tgt.sr + t * a.tgt.sc);
    const bool tgt_ok = tgt >= 0 && tgt < a.V;
    const int64_t tgt_safe = tgt_ok ? tgt : 0;  // never address outside the row
    // rrl_logprob_fwd_masked: a row whose mask is exactly 0 is never read.
    const bool fwd_skip = MODE == MODE_FWD && a.mask.ptr != nullptr && !a.mask.truth(b, t);
    // A row without a valid target (NLL's ignored label; an out-of-range id,
    // which is flagged) takes xt = -inf: e_t = 0, so the log-sum-exp stays the
    // row's own and its gradient row is exact (zeros when g = 0); its log-prob
    // is set to NaN below.
    const Acc xt = tgt_ok && !fwd_skip ? Tag::cvt(row[tgt_safe]) : -M<Acc>::inf();

    Acc lse, g, logp;
    bool have_logp = true;
    if (MODE == MODE_BWD) {
      lse = static_cast<const Acc*>(a.lse)[r];
      g = static_cast<const Acc*>(a.g)[r];
      have_logp = a.logp_in != nullptr;
      logp = have_logp ? static_cast<const Acc*>(a.logp_in)[r] : Acc(0);
      if (threadIdx.x == 0 && !tgt_ok) raise_flag(a.status, RRL_FLAG_TARGET_RANGE);
    } else if (fwd_skip) {
      // logp and lse written as 0; a target id outside [0, V) is still flagged.
      lse = Acc(0);
      logp = Acc(0);
      g = Acc(0);
      if (threadIdx.x == 0) {
        if (!tgt_ok) raise_flag(a.status, RRL_FLAG_TARGET_RANGE);
        store_as<Acc>(a.logp, a.logp_dt, r, logp);
        static_cast<Acc*>(a.lse_out)[r] = lse;
      }
    } else if (MODE == MODE_FUSED && (a.pp.flags & RRL_POLICY_SKIP_MASKED) &&
               weight_coef(mask_weight<Acc>(PolicyConsts<Acc>::make(a.pp), a.mask, b, t),
                           static_cast<const Acc*>(a.row_coef)[b]) == Acc(0)) {
      // Zero-weight row under RRL_POLICY_SKIP_MASKED: never read.
      lse = Acc(0);
      logp = Acc(0);
      g = Acc(0);
      if (threadIdx.x == 0) {
        if (!tgt_ok && !target_ignored(PolicyConsts<Acc>::make(a.pp), tgt))
          raise_flag(a.status, RRL_FLAG_TARGET_RANGE);
        store_as<Acc>(a.logp, a.logp_dt, r, logp);
        static_cast<Acc*>(a.lse_out)[r] = lse;
      }
    } else {
      // Sweep 1: online max / sum of exp over the non-target columns.
      Acc m = -M<Acc>::inf(), s = Acc(0);
      for (int64_t i = threadIdx.x; i < sp.head; i += NT) {
        Acc x[1] = {Tag::cvt(row[i])};
        online_update<Acc, 1>(m, s, x, i == tgt ? 0 : -1);
      }
      const S* body = row + sp.head;
      for (int64_t k = threadIdx.x; k < sp.nvec; k += NT) {
        Acc x[VEC];
        Tag::load_vec(body + k * VEC, x);
        const int64_t rel = tgt - (sp.head + k * VEC);
        online_update<Acc, VEC>(m, s, x, (rel >= 0 && rel < VEC) ? (int)rel : -1);
      }
      const int64_t tail0 = sp.head + sp.nvec * VEC;
      for (int64_t i = threadIdx.x; i < sp.tail; i += NT) {
        Acc x[1] = {Tag::cvt(row[tail0 + i])};
        online_update<Acc, 1>(m, s, x, tail0 + i == tgt ? 0 : -1);
      }
      block_online_combine<NT, Acc>(m, s, sh_m, sh_s);
      const RowLogprob<Acc> fr = finish_row<Acc>(m, s, xt);
      lse = fr.lse;
      logp = fr.logp;
      if (!tgt_ok) logp = M<Acc>::nan();
      g = Acc(0);
      if (MODE == MODE_FUSED) {
        const PolicyConsts<Acc> c = PolicyConsts<Acc>::make(a.pp);
        const Acc o = a.old.get<Acc>(b, t);
        const Acc A = a.adv.get<Acc>(b, t);
        const Acc w = mask_weight<Acc>(c, a.mask, b, t);
        const Acc coef = static_cast<const Acc*>(a.row_coef)[b];
        // loss = -objective, so dlogits carries d(-objective)/d logp.
        g = -(weight_coef(w, coef) * token_local_grad<Acc>(c, logp, o, A));
      }
      if (threadIdx.x == 0) {
        if (!tgt_ok && !(MODE == MODE_FUSED && target_ignored(PolicyConsts<Acc>::make(a.pp), tgt)))
          raise_flag(a.status, RRL_FLAG_TARGET_RANGE);
        store_as<Acc>(a.logp, a.logp_dt, r, logp);
        static_cast<Acc*>(a.lse_out)[r] = lse;
      }
    }

    if (MODE == MODE_BWD || MODE == MODE_FUSED) {
      // Sweep 2: dlogits = g * ([v == target] - exp(x - lse)).
      void* drow = static_cast<char*>(a.dl) +
                   (b * a.ds_b + t * a.ds_t) * (int64_t)dtype_size_dev(a.dl_dt);
      const bool zero_row = (g == Acc(0)) && (lse - lse == Acc(0));
      if (!(zero_row && a.accumulate)) {
        const Acc tgt_d = target_grad<Acc>(g, logp, have_logp, xt, lse);
        write_row_grad<Tag, NT>(row, sp, drow, a.dl_dt, a.V, tgt, g, lse, tgt_d, zero_row,
                                a.accumulate);
      }
    }
  }
}

template <class Tag, int MODE>
int launch_row(const RowArgs& a, hipStream_t stream) {
  constexpr int NT = 256;
  const int64_t rows = a.B * a.T;
  if (rows == 0) return RRL_OK;
  // A conditional rerun mostly returns at once: a grid of 2048 workgroups
  // keeps that launch short and still streams every row when it does run.
  const int64_t cap = (MODE == MODE_FUSED && (a.pp.flags & RRL_POLICY_RERUN_FAST_RANGE))
                          ? (int64_t)2048 : (int64_t)(1 << 30);
  const int64_t grid = rows < cap ? rows : cap;
  hipLaunchKernelGGL((row_kernel<Tag, MODE, NT>), dim3((unsigned)grid), dim3(NT), 0, stream, a);
  return check_launch("row_kernel");
}

template <int MODE>
int dispatch_row(const RowArgs& a, int logits_dtype, hipStream_t stream) {
  switch (logits_dtype) {
    case RRL_BF16: return launch_row<TagBF16, MODE>(a, stream);
    case RRL_F16: return launch_row<TagF16, MODE>(a, stream);
    case RRL_F32: return launch_row<TagF32, MODE>(a, stream);
    case RRL_F64: return launch_row<TagF64, MODE>(a, stream);
    default: set_error("logits dtype must be float32, float64, bfloat16 or float16"); return RRL_EDTYPE;
  }
}

// dlogits *= scale unless scale == skip_if: the single-pass kernel stores
// dlogits for d loss = 1, and autograd's upstream gradient is almost always 1,
// so this launch normally returns without touching memory.
template <typename Acc>
__global__ __launch_bounds__(256) void scale_rows_kernel(void* dl, int dt, int64_t B, int64_t T,
                                                         int64_t V, int64_t ds_b, int64_t ds_t,
                                                         const void* scale, int sdt, double skip_if) {
  const Acc s = load_as<Acc>(scale, sdt, 0);
  if ((double)s == skip_if) return;
  const int esz = dtype_size_dev(dt);
  for (int64_t r = blockIdx.x; r < B * T; r += gridDim.x) {
    const int64_t b = r / T, t = r - (r / T) * T;
    void* row = static_cast<char*>(dl) + (b * ds_b + t * ds_t) * (int64_t)esz;
    for (int64_t v = threadIdx.x; v < V; v += 256) store_as<Acc>(row, dt, v, load_as<Acc>(row, dt, v) * s);
  }
}

int validate_logits(const void* logits, int dt, int64_t B, int64_t T, int64_t V, rrl_view tgt) {
  RRL_REQUIRE(B >= 0 && T >= 0 && V >= 1, RRL_EINVAL, "logits sizes must be B>=0, T>=0, V>=1");
  RRL_REQUIRE(is_float_dtype(dt), RRL_EDTYPE, "logits dtype must be floating point");
  RRL_REQUIRE(B * T == 0 || logits != nullptr, RRL_EINVAL, "logits pointer is null");
  RRL_REQUIRE(B * T == 0 || tgt.ptr != nullptr, RRL_EINVAL, "targets pointer is null");
  RRL_REQUIRE(tgt.dtype == RRL_I32 || tgt.dtype == RRL_I64, RRL_EDTYPE,
              "target_ids must be int32 or int64");
  RRL_REQUIRE(((uintptr_t)logits % dtype_size(dt)) == 0, RRL_EALIGN, "logits pointer misaligned");
  return RRL_OK;
}

}  // namespace

int maybe_launch_resident(const RowArgs& a, int mode, int logits_dtype, hipStream_t stream,
                          bool* launched);

}  // namespace rrl

using namespace rrl;

extern "C" int rrl_logprob_fwd(const void* logits, int32_t logits_dtype, int64_t B, int64_t T,
                               int64_t V, int64_t ls_b, int64_t ls_t, rrl_view targets,
                               void* logp_out, int32_t logp_dtype, void* lse_out,
                               int32_t* status, void* stream) {
  clear_error();
  int rc = validate_logits(logits, logits_dtype, B, T, V, targets);
  if (rc) return rc;
  const int acc = logits_dtype == RRL_F64 ? RRL_F64 : RRL_F32;
  RRL_REQUIRE(logp_dtype == RRL_F32 || logp_dtype == RRL_F64, RRL_EDTYPE,
              "logp dtype must be float32 or float64");
  RRL_REQUIRE(B * T == 0 || (logp_out && lse_out), RRL_EINVAL, "null output pointer");
  (void)acc;
  RowArgs a{};
  a.logits = logits; a.B = B; a.T = T; a.V = V; a.ls_b = ls_b; a.ls_t = ls_t;
  a.tgt = to_view(targets);
  a.logp = logp_out; a.logp_dt = logp_dtype; a.lse_out = lse_out;
  a.status = status;
  return dispatch_row<MODE_FWD>(a, logits_dtype, as_stream(stream));
}

extern "C" int rrl_logprob_fwd_masked(const void* logits, int32_t logits_dtype, int64_t B,
                                      int64_t T, int64_t V, int64_t ls_b, int64_t ls_t,
                                      rrl_view targets, rrl_view mask, void* logp_out,
                                      int32_t logp_dtype, void* lse_out, int32_t* status,
                                      void* stream) {
  clear_error();
  int rc = validate_logits(logits, logits_dtype, B, T, V, targets);
  if (rc) return rc;
  RRL_REQUIRE(logp_dtype == RRL_F32 || logp_dtype == RRL_F64, RRL_EDTYPE,
              "logp dtype must be float32 or float64");
  RRL_REQUIRE(B * T == 0 || (logp_out && lse_out && mask.ptr), RRL_EINVAL,
              "null pointer argument");
  RowArgs a{};
  a.logits = logits; a.B = B; a.T = T; a.V = V; a.ls_b = ls_b; a.ls_t = ls_t;
  a.tgt = to_view(targets);
  a.mask = to_view(mask);
  a.logp = logp_out; a.logp_dt = logp_dtype; a.lse_out = lse_out;
  a.status = status;
  return dispatch_row<MODE_FWD>(a, logits_dtype, as_stream(stream));
}

extern "C" int rrl_logprob_bwd(const void* logits, int32_t logits_dtype, int64_t B, int64_t T,
                               int64_t V, int64_t ls_b, int64_t ls_t, rrl_view targets,
                               const void* lse, const void* logp, const void* g, void* dlogits,
                               int32_t dl_dtype, int64_t ds_b, int64_t ds_t, int32_t accumulate,
                               void* stream) {
  clear_error();
  int rc = validate_logits(logits, logits_dtype, B, T, V, targets);
  if (rc) return rc;
  RRL_REQUIRE(is_float_dtype(dl_dtype), RRL_EDTYPE, "dlogits dtype must be floating point");
  RRL_REQUIRE(B * T == 0 || (lse && g && dlogits), RRL_EINVAL, "null pointer argument");
  RowArgs a{};
  a.logits = logits; a.B = B; a.T = T; a.V = V; a.ls_b = ls_b; a.ls_t = ls_t;
  a.tgt = to_view(targets);
  a.lse = lse; a.logp_in = logp; a.g = g; a.dl = dlogits; a.dl_dt = dl_dtype; a.ds_b = ds_b; a.ds_t = ds_t;
  a.accumulate = accumulate;
  bool launched = false;
  rc = maybe_launch_resident(a, 1, logits_dtype, as_stream(stream), &launched);
  if (rc || launched) return rc;
  return dispatch_row<MODE_BWD>(a, logits_dtype, as_stream(stream));
}

namespace {

int fused_logprob_policy(const rrl_policy_params* params, const void* logits,
                         int32_t logits_dtype, int64_t B, int64_t T, int64_t V, int64_t ls_b,
                         int64_t ls_t, rrl_view targets, rrl_view old, rrl_view adv,
                         rrl_view mask, const void* row_coef, void* records, void* logp_out,
                         void* lse_out, void* dlogits, int32_t dl_dtype, int64_t ds_b,
                         int64_t ds_t, int32_t* status, void* stream) {
  RRL_REQUIRE(params != nullptr, RRL_EINVAL, "params is null");
  RRL_REQUIRE(params->kind == RRL_OBJ_PPO || params->kind == RRL_OBJ_SAO ||
                  params->kind == RRL_OBJ_SAPO || params->kind == RRL_OBJ_NLL,
              RRL_EINVAL,
              "single-pass path supports the token-local objectives PPO, SAO, SAPO, NLL");
  int rc = validate_logits(logits, logits_dtype, B, T, V, targets);
  if (rc) return rc;
  RRL_REQUIRE(is_float_dtype(dl_dtype), RRL_EDTYPE, "dlogits dtype must be floating point");
  RRL_REQUIRE(B * T == 0 || (logp_out && lse_out && dlogits && row_coef && old.ptr && adv.ptr &&
                             mask.ptr),
              RRL_EINVAL, "null pointer argument");
  RRL_REQUIRE(is_float_dtype(old.dtype) && is_float_dtype(adv.dtype), RRL_EDTYPE,
              "old log-probs and advantages must be floating point");
  RRL_REQUIRE(is_known_dtype(mask.dtype), RRL_EDTYPE, "unsupported mask dtype");
  RRL_REQUIRE(params->kind != RRL_OBJ_NLL || mask.dtype == RRL_I32 || mask.dtype == RRL_I64,
              RRL_EDTYPE, "NLL: the mask operand holds the target ids (int32 or int64)");
  RowArgs a{};
  a.logits = logits; a.B = B; a.T = T; a.V = V; a.ls_b = ls_b; a.ls_t = ls_t;
  a.tgt = to_view(targets);
  a.logp = logp_out; a.logp_dt = logits_dtype == RRL_F64 ? RRL_F64 : RRL_F32;
  a.lse_out = lse_out;
  a.dl = dlogits; a.dl_dt = dl_dtype; a.ds_b = ds_b; a.ds_t = ds_t;
  a.pp = *params; a.old = to_view(old); a.adv = to_view(adv); a.mask = to_view(mask);
  a.row_coef = row_coef; a.records = records; a.status = status;
  if (params->flags & RRL_POLICY_RERUN_FAST_RANGE) {
    RRL_REQUIRE(status != nullptr, RRL_EINVAL,
                "RRL_POLICY_RERUN_FAST_RANGE needs the first call's status word");
    return dispatch_row<MODE_FUSED>(a, logits_dtype, as_stream(stream));
  }
  bool launched = false;
  rc = maybe_launch_resident(a, 2, logits_dtype, as_stream(stream), &launched);
  if (rc || launched) return rc;
  return dispatch_row<MODE_FUSED>(a, logits_dtype, as_stream(stream));
}

// Records of rrl_fused_logprob_policy_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address); it passes the address hipGetSymbolAddress returns for the current
// device, looked up once per device and kept in g_scratch_addr.
static __device__ __align__(256) TokenRecord scratch[RRL_NOALLOC_MAX_TOKENS];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  RRL_REQUIRE(e == hipSuccess, RRL_ELAUNCH,
              std::string("hipGetDevice: ") + hipGetErrorString(e));
  RRL_REQUIRE(dev >= 0 && dev < kMaxDevices, RRL_EINVAL, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t se = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    RRL_REQUIRE(se == hipSuccess && p != nullptr, RRL_ELAUNCH,
                std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(se));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return RRL_OK;
}

}  // namespace

extern "C" int rrl_fused_logprob_policy(const rrl_policy_params* params, const void* logits,
                                        int32_t logits_dtype, int64_t B, int64_t T, int64_t V,
                                        int64_t ls_b, int64_t ls_t, rrl_view targets,
                                        rrl_view old, rrl_view adv, rrl_view mask,
                                        const void* row_coef, void* records, void* logp_out,
                                        void* lse_out, void* dlogits, int32_t dl_dtype,
                                        int64_t ds_b, int64_t ds_t, int32_t* status,
                                        void* stream) {
  clear_error();
  return fused_logprob_policy(params, logits, logits_dtype, B, T, V, ls_b, ls_t, targets, old,
                              adv, mask, row_coef, records, logp_out, lse_out, dlogits, dl_dtype,
                              ds_b, ds_t, status, stream);
}

extern "C" int rrl_fused_logprob_policy_noalloc(
    const rrl_policy_params* params, const void* logits, int32_t logits_dtype, int64_t B,
    int64_t T, int64_t V, int64_t ls_b, int64_t ls_t, rrl_view targets, rrl_view old,
    rrl_view adv, rrl_view mask, const void* row_coef, void* logp_out, void* lse_out,
    void* dlogits, int32_t dl_dtype, int64_t ds_b, int64_t ds_t, int32_t* status,
    void* stream) {
  clear_error();
  RRL_REQUIRE(B >= 0 && T >= 0, RRL_EINVAL, "negative size");
  RRL_REQUIRE(B * T <= (int64_t)RRL_NOALLOC_MAX_TOKENS, RRL_EINVAL,
              "rrl_fused_logprob_policy_noalloc: B*T = " + std::to_string(B * T) +
                  " tokens exceeds the static scratch of " +
                  std::to_string((int64_t)RRL_NOALLOC_MAX_TOKENS) +
                  " tokens; call rrl_fused_logprob_policy with a records workspace");
  void* records = nullptr;
  if (int rc = scratch_of_current_device(&records)) return rc;
  // Every record a sweep reads is written first by the same call's packing
  // kernel, so nothing in the array needs clearing between calls.
  return fused_logprob_policy(params, logits, logits_dtype, B, T, V, ls_b, ls_t, targets, old,
                              adv, mask, row_coef, records, logp_out, lse_out, dlogits, dl_dtype,
                              ds_b, ds_t, status, stream);
}

extern "C" size_t rrl_fused_records_bytes(int64_t B, int64_t T) {
  return (size_t)(B * T > 0 ? B * T : 0) * sizeof(TokenRecord) + 256;
}

extern "C" int rrl_scale_rows(void* dlogits, int32_t dl_dtype, int64_t B, int64_t T, int64_t V,
                              int64_t ds_b, int64_t ds_t, const void* scale, int32_t scale_dtype,
                              double skip_if, void* stream) {
  clear_error();
  RRL_REQUIRE(is_float_dtype(dl_dtype) && is_float_dtype(scale_dtype), RRL_EDTYPE,
              "dlogits and scale must be floating point");
  RRL_REQUIRE(B >= 0 && T >= 0 && V >= 0, RRL_EINVAL, "negative size");
  if (B * T * V == 0) return RRL_OK;
  RRL_REQUIRE(dlogits && scale, RRL_EINVAL, "null pointer argument");
  const int64_t rows = B * T;
  // Mostly a launch that returns at once (scale == skip_if): 4096 workgroups
  // keep it at a few microseconds, where one per row took 56 us at 262144
  // rows, and still cover every row when it does scale.
  const unsigned grid = (unsigned)(rows < 4096 ? rows : 4096);
  hipStream_t st = as_stream(stream);
  if (dl_dtype == RRL_F64 || scale_dtype == RRL_F64)
    hipLaunchKernelGGL((scale_rows_kernel<double>), dim3(grid), dim3(256), 0, st, dlogits,
                       (int)dl_dtype, B, T, V, ds_b, ds_t, scale, (int)scale_dtype, skip_if);
  else
    hipLaunchKernelGGL((scale_rows_kernel<float>), dim3(grid), dim3(256), 0, st, dlogits,
                       (int)dl_dtype, B, T, V, ds_b, ds_t, scale, (int)scale_dtype, skip_if);
  return check_launch("scale_rows_kernel");
}
