// Register-resident 16-bit row kernels: the fast path of
// rrl_fused_logprob_policy (log-prob + token-local objective gradient in one
// read of the logits, losses.py:14-38 composed with :426-486 / :127-203 /
// :355-423), and of rrl_logprob_bwd (resident_bwd_kernel, the backward of
// losses.py:34-38 given the forward's lse and log-probs).
//
// Layout and schedule (gfx950, wave64):
//   * A persistent grid of one 1024-lane workgroup per CU walks rows
//     r = blockIdx.x, blockIdx.x + gridDim.x, ...
//   * A row of V 16-bit logits is held in VGPRs as SL slabs of one 16-byte
//     vector per lane: slab k, lane j holds vector k*1024 + j.  V = 151936
//     (bf16) is 18992 vectors, SL = 19 of the SL = 20 variant, i.e. 80 VGPRs.
//   * Per-row scalars (target, old log-prob, advantage, mask weight * 1/M)
//     come from a packed 16-byte record per token (pack_records_kernel), read
//     a row ahead through the scalar cache.
//   * Sweep 1 (registers only): online max / sum of exp over the non-target
//     columns per lane, slab by slab as the loads land, then one LDS combine
//     across the 16 waves.
//   * Sweep 2: each slab becomes g * (onehot - exp(x - lse)), is packed back to
//     16 bits and stored with a non-temporal buffer store; once the whole row
//     is stored, the same registers are refilled with the workgroup's next
//     row, so the next row's HBM reads overlap the drain of this row's stores.
// Every access is a raw buffer load/store whose descriptor covers exactly one
// row, so a lane past the end of the row reads zeros and its stores are
// dropped by the hardware range check.
#include <hip/hip_runtime.h>

#include "policy_math.hpp"
#include "row_common.hpp"
#include "wave_common.hpp"

namespace rrl {

namespace {

constexpr int RNT = 1024;                 // lanes per workgroup (16 waves)

// Element access of one 16-byte vector per tag: EPV elements, their float
// values, the packed form written back (round to nearest even for 16-bit),
// the sign bit of every element of a dword, and the single-element loads and
// non-temporal stores of a row's unaligned head and tail.
template <class Tag> struct Pack16;
template <> struct Pack16<TagBF16> {
  static constexpr int EPV = 8, LOG2_EPV = 3;
  static constexpr uint32_t SGN2 = 0x80008000u, SGN1 = 0x8000u;
  static __device__ __forceinline__ void unpack(const u32x4& u, float (&x)[8]) {
    x[0] = __uint_as_float(u.x << 16); x[1] = __uint_as_float(u.x & 0xffff0000u);
    x[2] = __uint_as_float(u.y << 16); x[3] = __uint_as_float(u.y & 0xffff0000u);
    x[4] = __uint_as_float(u.z << 16); x[5] = __uint_as_float(u.z & 0xffff0000u);
    x[6] = __uint_as_float(u.w << 16); x[7] = __uint_as_float(u.w & 0xffff0000u);
  }
  static __device__ __forceinline__ u32x4 pack(const float (&d)[8]) {
    u32x4 o;
    o.x = f32x2_to_bf16x2_bits(d[0], d[1]);
    o.y = f32x2_to_bf16x2_bits(d[2], d[3]);
    o.z = f32x2_to_bf16x2_bits(d[4], d[5]);
    o.w = f32x2_to_bf16x2_bits(d[6], d[7]);
    return o;
  }
  static __device__ __forceinline__ float one(uint32_t b) { return __uint_as_float(b << 16); }
  static __device__ __forceinline__ uint32_t pack_one(float d) { return f32_to_bf16_bits(d); }
  static __device__ __forceinline__ uint32_t load_one(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
  static __device__ __forceinline__ void store_one(uint32_t b, __amdgpu_buffer_rsrc_t r, int off) {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)b, r, off, 0, kAuxStoreNT);
  }
};
template <> struct Pack16<TagF16> {
  static constexpr int EPV = 8, LOG2_EPV = 3;
  static constexpr uint32_t SGN2 = 0x80008000u, SGN1 = 0x8000u;
  static __device__ __forceinline__ void unpack(const u32x4& u, float (&x)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = f16_bits_to_f32((uint16_t)(w[i] & 0xffffu));
      x[2 * i + 1] = f16_bits_to_f32((uint16_t)(w[i] >> 16));
    }
  }
  static __device__ __forceinline__ u32x4 pack(const float (&d)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)f32_to_f16_bits(d[2 * i]) | ((uint32_t)f32_to_f16_bits(d[2 * i + 1]) << 16);
    u32x4 o;
    o.x = w[0]; o.y = w[1]; o.z = w[2]; o.w = w[3];
    return o;
  }
  static __device__ __forceinline__ float one(uint32_t b) {
    return f16_bits_to_f32((uint16_t)(b & 0xffffu));
  }
  static __device__ __forceinline__ uint32_t pack_one(float d) { return f32_to_f16_bits(d); }
  static __device__ __forceinline__ uint32_t load_one(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
  static __device__ __forceinline__ void store_one(uint32_t b, __amdgpu_buffer_rsrc_t r, int off) {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)b, r, off, 0, kAuxStoreNT);
  }
};
template <> struct Pack16<TagF32> {
  static constexpr int EPV = 4, LOG2_EPV = 2;
  static constexpr uint32_t SGN2 = 0x80000000u, SGN1 = 0x80000000u;
  static __device__ __forceinline__ void unpack(const u32x4& u, float (&x)[4]) {
    x[0] = __uint_as_float(u.x); x[1] = __uint_as_float(u.y);
    x[2] = __uint_as_float(u.z); x[3] = __uint_as_float(u.w);
  }
  static __device__ __forceinline__ u32x4 pack(const float (&d)[4]) {
    u32x4 o;
    o.x = __float_as_uint(d[0]); o.y = __float_as_uint(d[1]);
    o.z = __float_as_uint(d[2]); o.w = __float_as_uint(d[3]);
    return o;
  }
  static __device__ __forceinline__ float one(uint32_t b) { return __uint_as_float(b); }
  static __device__ __forceinline__ uint32_t pack_one(float d) { return __float_as_uint(d); }
  static __device__ __forceinline__ uint32_t load_one(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  }
  static __device__ __forceinline__ void store_one(uint32_t b, __amdgpu_buffer_rsrc_t r, int off) {
    __builtin_amdgcn_raw_buffer_store_b32(b, r, off, 0, kAuxStoreNT);
  }
};

// A row as the resident kernels hold it: `head` single elements up to the
// first 128-byte boundary, `nbody` 16-byte vectors (the register slabs), then
// `tail` single elements.  The body starts on a 128-byte boundary so that
// each wave's 1 KB run of vector stores covers whole cache lines: runs that
// share a partly written line with the next wave's run cost up to 10% of the
// write rate.  head < 128 / element size (at most 63) and tail <= EPV - 1,
// so lanes 0-63 carry the head and lanes 64-71 the tail in one extra
// register.  Without EXTRAS every row is 16-byte aligned with V % EPV == 0:
// head = tail = 0 and nbody is the same for every row.
constexpr uint32_t kBodyAlign = 128;
constexpr int kHeadLanes = 64;

struct RowGeo {
  uint32_t head, nbody, tail;
};

template <class Tag, bool EXTRAS>
__device__ __forceinline__ RowGeo row_geo(const void* row, uint32_t V, int32_t nvec) {
  constexpr uint32_t EPV = Pack16<Tag>::EPV, ESZ = 16 / EPV;
  RowGeo g;
  if constexpr (EXTRAS) {
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(row) & (kBodyAlign - 1u));
    uint32_t h = mis ? (kBodyAlign - mis) / ESZ : 0u;
    h = h < V ? h : V;
    const uint32_t rem = V - h;
    g.head = h;
    g.nbody = rem / EPV;
    g.tail = rem - g.nbody * EPV;
  } else {
    g.head = 0;
    g.nbody = (uint32_t)nvec;
    g.tail = 0;
  }
  return g;
}

// Vocabulary index of the extra element lane `tid` carries, or -1.
template <class Tag>
__device__ __forceinline__ int32_t extra_index(const RowGeo& g, int tid) {
  constexpr int EPV = Pack16<Tag>::EPV;
  if (tid < kHeadLanes) return tid < (int)g.head ? tid : -1;
  if (tid < kHeadLanes + EPV)
    return tid - kHeadLanes < (int)g.tail ? (int)(g.head + g.nbody * EPV) + tid - kHeadLanes : -1;
  return -1;
}

// Per-token records for the resident kernel (TokenRecord): the views' dtype
// and stride handling happens here, once per token, so that the row loop reads
// its scalars with one uniform 16-byte load.
__global__ __launch_bounds__(256) void pack_records_kernel(RowArgs a) {
  const PolicyConsts<float> c = PolicyConsts<float>::make(a.pp);
  TokenRecord* rec = static_cast<TokenRecord*>(a.records);
  const float* coef = static_cast<const float*>(a.row_coef);
  const int64_t n = a.B * a.T;
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t b = i / a.T, t = i - (i / a.T) * a.T;
    const int64_t tgt = load_index(a.tgt.ptr, a.tgt.dt, b * a.tgt.sr + t * a.tgt.sc);
    const bool ok = tgt >= 0 && tgt < a.V;
    if (!ok && !target_ignored(c, tgt)) raise_flag(a.status, RRL_FLAG_TARGET_RANGE);
    TokenRecord r;
    r.target = ok ? (int32_t)tgt : -1;
    r.old = a.old.get<float>(b, t);
    r.adv = a.adv.get<float>(b, t);
    r.wcoef = weight_coef(mask_weight<float>(c, a.mask, b, t), coef[b]);
    rec[i] = r;
  }
}

// The records are read-only for the resident kernel, so they can come through
// the scalar data cache: a uniform load from the constant address space is a
// single s_load_dwordx4, waited on with lgkmcnt and never behind the
// vector-memory queue of slab loads and stores.
__device__ __forceinline__ TokenRecord load_record(const void* base, uint32_t r) {
  typedef __attribute__((address_space(4))) const u32x4 ConstWords;
  const u32x4 q = reinterpret_cast<ConstWords*>(reinterpret_cast<uintptr_t>(base))[r];
  TokenRecord rec;
  rec.target = (int32_t)q.x;
  rec.old = __uint_as_float(q.y);
  rec.adv = __uint_as_float(q.z);
  rec.wcoef = __uint_as_float(q.w);
  return rec;
}

// s * exp(m - M) for the combine: exact s when m == M (also for M = -inf or
// +inf, where m - M is NaN), 0 for m = -inf below a finite M.
__device__ __forceinline__ float rescale(float s, float m, float M) {
  return m == M ? s : s * exp2_hw((m - M) * kLog2e);
}

// Balanced max / sum of the EPV values of one vector.
template <int N>
__device__ __forceinline__ float vmax(const float (&v)[N]) {
  if constexpr (N == 8)
    return fmaxf(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])),
                 fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
  else
    return fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
}
template <int N>
__device__ __forceinline__ float vsum(const float (&e)[N]) {
  if constexpr (N == 8)
    return ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
  else
    return (e[0] + e[1]) + (e[2] + e[3]);
}

// exp2 exponent of -g * exp(x - lse) without the sign: x*log2e + (log2|g| -
// lse*log2e) for 16-bit logits (one FMA per element; |lse| > 2e38 is flagged
// and rerun by the host), (x - lse)*log2e + log2|g| for float32 logits (a
// subtract more, and exact for every finite lse).
struct ExpArg {
  float cg, lg, lse;
};
template <class Tag>
__device__ __forceinline__ float exp_arg(float x, const ExpArg& q) {
  if constexpr (Pack16<Tag>::EPV == 4)
    return __builtin_fmaf(x - q.lse, kLog2e, q.lg);
  else
    return __builtin_fmaf(x, kLog2e, q.cg);
}

template <class Tag, int SL, bool EXTRAS>
__global__ __launch_bounds__(RNT) void resident_fused_kernel(RowArgs a, int32_t nvec) {
  using P = Pack16<Tag>;
  using S = typename Tag::S;
  constexpr int EPV = P::EPV;
  constexpr int ESZ = (int)sizeof(S);
  // Double-buffered by combine parity: a wave can run at most one combine
  // ahead of the slowest (each combine has one barrier), so the buffer it
  // writes is never the one another wave is still reading.
  __shared__ float sh_m[2][RNT / 64];
  __shared__ float sh_s[2][RNT / 64];
  __shared__ float sh_xt[2];
  int buf = 0;

  const int tid = threadIdx.x;
  const int64_t rows = a.B * a.T;
  const uint32_t V32 = (uint32_t)a.V;
  const int voff = tid * 16;
  const S* logits = static_cast<const S*>(a.logits);
  S* dl = static_cast<S*>(a.dl);
  const PolicyConsts<float> c = PolicyConsts<float>::make(a.pp);
  // Row indices fit in 32 bits (checked on the host); 32-bit division keeps the
  // per-row address arithmetic short.
  const uint32_t T32 = (uint32_t)a.T;
  const uint32_t rows32 = (uint32_t)rows;
  uint32_t r = blockIdx.x;
  if (r >= rows32) return;

  auto row_ptr = [&](uint32_t rr) {
    const uint32_t bb = rr / T32, tt = rr - bb * T32;
    return logits + (int64_t)bb * a.ls_b + (int64_t)tt * a.ls_t;
  };
  // The extra element of this lane (EXTRAS): its byte offset in the row, or
  // the row's end (out of range: loads return 0, stores are dropped).
  auto extra_off = [&](const RowGeo& g) {
    const int32_t ei = extra_index<Tag>(g, tid);
    return ei >= 0 ? ei * ESZ : (int)(V32 * ESZ);
  };
  // RRL_POLICY_SKIP_MASKED: rows whose weight is exactly 0 are never read
  // (their loads use a 0-byte descriptor: no memory traffic) and get zero
  // dlogits and log-prob 0.
  const bool skip_masked = (a.pp.flags & RRL_POLICY_SKIP_MASKED) != 0;
  TokenRecord rec_next = load_record(a.records, r);
  u32x4 x[SL];
  uint32_t xe = 0;  // EXTRAS: the lane's head or tail element, as stored
  {
    const bool skip0 = skip_masked && rec_next.wcoef == 0.0f;
    const S* p0 = row_ptr(r);
    const RowGeo g0 = row_geo<Tag, EXTRAS>(p0, V32, nvec);
    const __amdgpu_buffer_rsrc_t src = skip0 ? row_rsrc(logits, 0u) : row_rsrc(p0 + g0.head, g0.nbody * 16);
    // Issue in slab order, the order sweep 2 refills them: with one order on
    // both paths into the row loop, sweep 1 waits for slab k only (older
    // loads), not for the whole row.
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      x[k] = __builtin_amdgcn_raw_buffer_load_b128(src, voff, k * RNT * 16, kAuxLoad);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EXTRAS) {
      const __amdgpu_buffer_rsrc_t esrc = skip0 ? row_rsrc(logits, 0u) : row_rsrc(p0, V32 * ESZ);
      xe = P::load_one(esrc, extra_off(g0));
    }
  }

  for (; r < rows32; r += gridDim.x) {
    const uint32_t b = r / T32, t = r - b * T32;
    // An opaque per-row copy of the lane id: the per-slab compares below are
    // then recomputed each row instead of being hoisted (and spilled) as 2*SL
    // loop-invariant masks.
    int lane = tid;
    asm volatile("" : "+v"(lane));
    const RowGeo g = row_geo<Tag, EXTRAS>(row_ptr(r), V32, nvec);
    const int32_t ei = EXTRAS ? extra_index<Tag>(g, tid) : -1;
    // Per-row scalars: one scalar-cache load, issued a row ahead.
    const TokenRecord rec = rec_next;
    const bool skip = skip_masked && rec.wcoef == 0.0f;
    const uint32_t rn = r + gridDim.x;
    const bool has_next = rn < rows32;
    if (has_next) rec_next = load_record(a.records, rn);
    const int32_t tgt = rec.target;
    const bool tgt_ok = tgt >= 0;
    // Slab k of this lane holds the target iff rel == k * RNT; a target in
    // the head or tail is the extra element of lane ei == tgt.
    const int32_t bt = tgt - (int32_t)g.head;
    const bool in_body = tgt_ok && (!EXTRAS || (bt >= 0 && bt < (int32_t)(g.nbody * EPV)));
    const int rel = in_body ? (bt >> P::LOG2_EPV) - lane : -1;
    const int ti = bt & (EPV - 1);
    const bool ex_tgt = EXTRAS && tgt_ok && ei == tgt;

    // Sweep 1: per-lane online (max, sum exp) over the slabs.  The running max
    // starts at -inf; `mg` (the max as an exponent offset) is kept finite so
    // that slabs of -inf contribute exp(-inf) = 0 rather than
    // exp(-inf + inf) = NaN, while NaN and +inf still poison the row as in
    // log_softmax.  The target column is left out of the sum in the one lane
    // and slab that hold it.
    float m = -__builtin_huge_valf(), s = 0.0f;
    auto fold = [&](int k) {
      if (lane < (int)g.nbody - k * RNT) {
        float v[EPV];
        P::unpack(x[k], v);
        const float mn = fmaxf(m, vmax(v));
        const float mg = fmaxf(mn, -__FLT_MAX__);
        float e[EPV];
#pragma unroll
        for (int i = 0; i < EPV; ++i) e[i] = exp2_hw((v[i] - mg) * kLog2e);
        float se = vsum(e);
        if (rel == k * RNT) {
          float xv = v[0], so = 0.0f;
#pragma unroll
          for (int i = 0; i < EPV; ++i) {
            xv = (i == ti) ? v[i] : xv;
            so += (i == ti) ? 0.0f : e[i];
          }
          se = so;
          sh_xt[buf] = xv;
        }
        s = __builtin_fmaf(s, exp2_hw((m - mg) * kLog2e), se);
        m = mn;
      }
    };
    float xt = 0.0f;
    if (!skip) {  // uniform over the workgroup
#pragma unroll
      for (int k = 0; k < SL; ++k) fold(k);
      if constexpr (EXTRAS) {
        // As in a slab: the element joins the max, and the sum unless it is
        // the target.
        if (ei >= 0) {
          const float v = P::one(xe);
          const float mn = fmaxf(m, v);
          const float mg = fmaxf(mn, -__FLT_MAX__);
          const float ev = ex_tgt ? 0.0f : exp2_hw((v - mg) * kLog2e);
          if (ex_tgt) sh_xt[buf] = v;
          s = __builtin_fmaf(s, exp2_hw((m - mg) * kLog2e), ev);
          m = mn;
        }
      }
      // No valid target: xt = -inf keeps the row's log-sum-exp finite (the
      // log-prob is set to NaN below).
      if (!tgt_ok && tid == 0) sh_xt[buf] = -__builtin_huge_valf();
      // Workgroup combine, kept short: the next row's loads are not issued
      // until it ends.  Wave max, then the rescaled sum (one exponential per
      // lane), then the 16 wave pairs through LDS with one barrier.
      const float Mw = wave_max_dpp(m);
      const float Sw = wave_sum_dpp(rescale(s, m, Mw));
      if ((tid & 63) == 0) {
        sh_m[buf][tid >> 6] = Mw;
        sh_s[buf][tid >> 6] = Sw;
      }
      lds_barrier();
      float mw[RNT / 64];
#pragma unroll
      for (int i = 0; i < RNT / 64; ++i) mw[i] = sh_m[buf][i];
      m = mw[0];
#pragma unroll
      for (int i = 1; i < RNT / 64; ++i) m = fmaxf(m, mw[i]);
      float sp[RNT / 64];
#pragma unroll
      for (int i = 0; i < RNT / 64; ++i) sp[i] = rescale(sh_s[buf][i], mw[i], m);
#pragma unroll
      for (int w = RNT / 128; w > 0; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) sp[i] += sp[i + w];
      s = sp[0];
      xt = sh_xt[buf];
      buf ^= 1;
    }
    // Past the last row (or for a skipped next row) the descriptor covers 0
    // bytes: the refills return zeros without touching memory.
    const bool skip_next = skip_masked && rec_next.wcoef == 0.0f;
    const bool load_next = has_next && !skip_next;
    const S* pn = row_ptr(load_next ? rn : r);
    const RowGeo gn = row_geo<Tag, EXTRAS>(pn, V32, nvec);
    const __amdgpu_buffer_rsrc_t src =
        load_next ? row_rsrc(pn + gn.head, gn.nbody * 16) : row_rsrc(logits, 0u);

    // Opaque to the optimiser: sweep 2 re-expands the packed slabs instead of
    // keeping sweep 1's widened copies live (twice the registers).
#pragma unroll
    for (int k = 0; k < SL; ++k) asm volatile("" : "+v"(x[k]));
    if constexpr (EXTRAS) asm volatile("" : "+v"(xe));

    const RowLogprob<float> fr = finish_row<float>(m, s, xt);
    const float lse = skip ? 0.0f : fr.lse;
    const float logp = skip ? 0.0f : (tgt_ok ? fr.logp : __builtin_nanf(""));
    const float gr =
        skip ? 0.0f : -(rec.wcoef * token_local_grad<float>(c, logp, rec.old, rec.adv));
    const float tgt_d = target_grad<float>(gr, logp, true, xt, lse);
    if (tid == 0) {
      store_as<float>(a.logp, a.logp_dt, r, logp);
      static_cast<float*>(a.lse_out)[r] = lse;
    }

    // Sweep 2: dlogits, then refill the register slabs with the next row.
    const S* drow = dl + (int64_t)b * a.ds_b + (int64_t)t * a.ds_t;
    const __amdgpu_buffer_rsrc_t dst = row_rsrc(drow + g.head, g.nbody * 16);
    // lse * log2e overflows for finite |lse| > 2.3e38 (logits near the 16-bit
    // maximum): such a row is flagged and the host reruns the call on the
    // generic kernel.  Non-finite lse needs no care: NaN propagates as in
    // log_softmax.  Float32 logits use the x - lse form, which has no limit.
    if (EPV == 8 && tid == 0 && fabsf(lse) > 2e38f && fabsf(lse) != __builtin_huge_valf())
      raise_flag(a.status, RRL_FLAG_FAST_RANGE);
    // -g * exp(x - lse) = -sign(g) * exp2(x*log2e + (log2|g| - lse*log2e)):
    // one FMA and one v_exp_f32 per element; the sign is applied to the packed
    // words with one XOR per dword.
    ExpArg q;
    q.lg = __log2f(fabsf(gr));
    q.cg = q.lg - lse * kLog2e;
    q.lse = lse;
    const bool flip = gr > 0.0f;
    const uint32_t sgn = flip ? P::SGN2 : 0u;
    const float tgt_pre = flip ? -tgt_d : tgt_d;  // the XOR restores tgt_d
    // Every element goes through the same arithmetic, also for a zero-weight
    // row: there log2|g| = -inf and exp2(-inf) = 0 for every finite or -inf
    // logit (a +inf or NaN logit makes lse non-finite and the row NaN, as in
    // log_softmax).  A uniform branch around the arithmetic with
    // zero-initialised registers was tried with the store-then-load order
    // below: on gfx950 it stored the zero initialiser instead of the computed
    // first dword of odd slabs in waves 4-15, so it is not used.
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      float d[EPV];
      float v[EPV];
      P::unpack(x[k], v);
#pragma unroll
      for (int i = 0; i < EPV; ++i) d[i] = exp2_hw(exp_arg<Tag>(v[i], q));
      if (rel == k * RNT) {
#pragma unroll
        for (int i = 0; i < EPV; ++i) d[i] = (i == ti) ? tgt_pre : d[i];
      }
      u32x4 o = P::pack(d);
      o.x ^= sgn; o.y ^= sgn; o.z ^= sgn; o.w ^= sgn;
      __builtin_amdgcn_raw_buffer_store_b128(o, dst, voff, k * RNT * 16, kAuxStoreNT);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EXTRAS) {
      const float dv = ex_tgt ? tgt_pre : exp2_hw(exp_arg<Tag>(P::one(xe), q));
      P::store_one(P::pack_one(dv) ^ (flip ? P::SGN1 : 0u), row_rsrc(drow, V32 * ESZ),
                   extra_off(g));
      __builtin_amdgcn_sched_barrier(0);
    }
    // Then the next row's loads into the same registers: each CU issues its
    // row's stores as one burst and the next row's loads as another instead
    // of alternating 16-byte stores and loads, which the memory system serves
    // 8-12% faster (5.7 against 5.1-5.3 TB/s for the same 1R + 1W bytes).
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      x[k] = __builtin_amdgcn_raw_buffer_load_b128(src, voff, k * RNT * 16, kAuxLoad);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EXTRAS) {
      const __amdgpu_buffer_rsrc_t esrc = load_next ? row_rsrc(pn, V32 * ESZ) : row_rsrc(logits, 0u);
      xe = P::load_one(esrc, extra_off(gn));
    }
  }
}

// Per-row inputs of the backward (rrl_logprob_bwd): target id, log-sum-exp,
// upstream gradient g = d loss / d logp and the forward's log-prob, each a
// uniform load through the scalar data cache (read-only in this kernel).
struct BwdRow {
  int64_t target;
  float lse, g, logp;
};

__device__ __forceinline__ BwdRow load_bwd_row(const RowArgs& a, uint32_t r, uint32_t T32) {
  typedef __attribute__((address_space(4))) const float CF;
  typedef __attribute__((address_space(4))) const int32_t CI32;
  typedef __attribute__((address_space(4))) const int64_t CI64;
  const uint32_t b = r / T32, t = r - b * T32;
  const int64_t off = (int64_t)b * a.tgt.sr + (int64_t)t * a.tgt.sc;
  const uintptr_t tp = reinterpret_cast<uintptr_t>(a.tgt.ptr);
  BwdRow q;
  q.target = a.tgt.dt == RRL_I32 ? (int64_t)reinterpret_cast<CI32*>(tp)[off]
                                 : reinterpret_cast<CI64*>(tp)[off];
  q.lse = reinterpret_cast<CF*>(reinterpret_cast<uintptr_t>(a.lse))[r];
  q.g = reinterpret_cast<CF*>(reinterpret_cast<uintptr_t>(a.g))[r];
  q.logp = reinterpret_cast<CF*>(reinterpret_cast<uintptr_t>(a.logp_in))[r];
  return q;
}

// A row whose gradient is exactly zero and whose log-sum-exp is finite has
// all-zero dlogits: its logits are never read.
__device__ __forceinline__ bool bwd_zero_row(const BwdRow& q) {
  return q.g == 0.0f && q.lse - q.lse == 0.0f;
}

// rrl_logprob_bwd for 16-bit and float32 rows (losses.py:34-38 backward):
// dlogits = g * (onehot(target) - exp(x - lse)) with lse, g and log-prob given,
// so there is no reduction and no exchange between lanes.  The schedule is the
// fused kernel's sweep 2: the row sits in VGPRs as SL slabs of 16 bytes per
// lane (plus the head and tail elements with EXTRAS), is written back as one
// burst of stores and the registers are refilled with the workgroup's next
// row as one burst of loads.  The waves never synchronise.
template <class Tag, int SL, bool EXTRAS>
__global__ __launch_bounds__(RNT) void resident_bwd_kernel(RowArgs a, int32_t nvec) {
  using P = Pack16<Tag>;
  using S = typename Tag::S;
  constexpr int EPV = P::EPV;
  constexpr int ESZ = (int)sizeof(S);
  const int tid = threadIdx.x;
  const uint32_t rows32 = (uint32_t)(a.B * a.T);
  const uint32_t T32 = (uint32_t)a.T;
  const uint32_t V32 = (uint32_t)a.V;
  const int voff = tid * 16;
  const S* logits = static_cast<const S*>(a.logits);
  S* dl = static_cast<S*>(a.dl);
  uint32_t r = blockIdx.x;
  if (r >= rows32) return;

  auto row_ptr = [&](uint32_t rr) {
    const uint32_t bb = rr / T32, tt = rr - bb * T32;
    return logits + (int64_t)bb * a.ls_b + (int64_t)tt * a.ls_t;
  };
  auto extra_off = [&](const RowGeo& g) {
    const int32_t ei = extra_index<Tag>(g, tid);
    return ei >= 0 ? ei * ESZ : (int)(V32 * ESZ);
  };
  BwdRow next = load_bwd_row(a, r, T32);
  u32x4 x[SL];
  uint32_t xe = 0;
  {
    const bool z0 = bwd_zero_row(next);
    const S* p0 = row_ptr(r);
    const RowGeo g0 = row_geo<Tag, EXTRAS>(p0, V32, nvec);
    const __amdgpu_buffer_rsrc_t src = z0 ? row_rsrc(logits, 0u) : row_rsrc(p0 + g0.head, g0.nbody * 16);
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      x[k] = __builtin_amdgcn_raw_buffer_load_b128(src, voff, k * RNT * 16, kAuxLoad);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EXTRAS)
      xe = P::load_one(z0 ? row_rsrc(logits, 0u) : row_rsrc(p0, V32 * ESZ), extra_off(g0));
  }

  // The zero rows' store data: a register quad of its own, opaque so that it
  // is not rematerialised into a slab register whose load is still pending
  // (that would make the zero stores wait on vmcnt, which on gfx9 also waits
  // for every older store to be acknowledged).
  u32x4 zv = {0u, 0u, 0u, 0u};
  asm volatile("" : "+v"(zv));

  for (; r < rows32; r += gridDim.x) {
    const uint32_t b = r / T32, t = r - b * T32;
    int lane = tid;
    asm volatile("" : "+v"(lane));
    const RowGeo g = row_geo<Tag, EXTRAS>(row_ptr(r), V32, nvec);
    const int32_t ei = EXTRAS ? extra_index<Tag>(g, tid) : -1;
    const BwdRow cur = next;
    const uint32_t rn = r + gridDim.x;
    const bool has_next = rn < rows32;
    if (has_next) next = load_bwd_row(a, rn, T32);
    // A target outside [0, V) has no column: every element takes the
    // exp(x - lse) term, as in the generic kernel.
    const bool tgt_ok = cur.target >= 0 && cur.target < a.V;
    const int32_t tgt = tgt_ok ? (int32_t)cur.target : 0;
    const int32_t bt = tgt - (int32_t)g.head;
    const bool in_body = tgt_ok && (!EXTRAS || (bt >= 0 && bt < (int32_t)(g.nbody * EPV)));
    const int rel = in_body ? (bt >> P::LOG2_EPV) - lane : -1;
    const int ti = bt & (EPV - 1);
    const bool ex_tgt = EXTRAS && tgt_ok && ei == tgt;
    const bool zero = bwd_zero_row(cur);
    const float gr = cur.g, lse = cur.lse;
    // -g * exp(x - lse) = -sign(g) * exp2((x - lse) * log2e + log2|g|): the
    // difference is formed first, so no finite lse overflows.
    const float lg = __log2f(fabsf(gr));
    const bool flip = gr > 0.0f;
    const uint32_t sgn = flip ? P::SGN2 : 0u;
    const float tgt_d = zero ? 0.0f : target_grad<float>(gr, cur.logp, true, 0.0f, lse);
    const float tgt_pre = flip ? -tgt_d : tgt_d;  // the XOR restores tgt_d
    const bool load_next = has_next && !bwd_zero_row(next);
    const S* pn = row_ptr(load_next ? rn : r);
    const RowGeo gn = row_geo<Tag, EXTRAS>(pn, V32, nvec);
    const __amdgpu_buffer_rsrc_t src =
        load_next ? row_rsrc(pn + gn.head, gn.nbody * 16) : row_rsrc(logits, 0u);
    const S* drow = dl + (int64_t)b * a.ds_b + (int64_t)t * a.ds_t;
    const __amdgpu_buffer_rsrc_t dst = row_rsrc(drow + g.head, g.nbody * 16);
    if (zero) {  // uniform over the workgroup
      // Stores only, with no dependence on the (never read) slabs: a run of
      // zero rows (a clipped GSPO sequence, masked prompt tokens) streams its
      // stores without waiting for earlier ones.  Measured on config 3 (72%
      // zero rows): backward 16.8-18.4 ms against 18.6-20.0 ms when the zero
      // rows went through the arithmetic below.
#pragma unroll
      for (int k = 0; k < SL; ++k) {
        __builtin_amdgcn_raw_buffer_store_b128(zv, dst, voff, k * RNT * 16, kAuxStoreNT);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (EXTRAS) {
        P::store_one(zv.x, row_rsrc(drow, V32 * ESZ), extra_off(g));
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int k = 0; k < SL; ++k) {
        float d[EPV];
        float v[EPV];
        P::unpack(x[k], v);
#pragma unroll
        for (int i = 0; i < EPV; ++i) d[i] = exp2_hw(__builtin_fmaf(v[i] - lse, kLog2e, lg));
        if (rel == k * RNT) {
#pragma unroll
          for (int i = 0; i < EPV; ++i) d[i] = (i == ti) ? tgt_pre : d[i];
        }
        u32x4 o = P::pack(d);
        o.x ^= sgn; o.y ^= sgn; o.z ^= sgn; o.w ^= sgn;
        __builtin_amdgcn_raw_buffer_store_b128(o, dst, voff, k * RNT * 16, kAuxStoreNT);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (EXTRAS) {
        const float dv =
            ex_tgt ? tgt_pre : exp2_hw(__builtin_fmaf(P::one(xe) - lse, kLog2e, lg));
        P::store_one(P::pack_one(dv) ^ (flip ? P::SGN1 : 0u), row_rsrc(drow, V32 * ESZ),
                     extra_off(g));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      x[k] = __builtin_amdgcn_raw_buffer_load_b128(src, voff, k * RNT * 16, kAuxLoad);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EXTRAS)
      xe = P::load_one(load_next ? row_rsrc(pn, V32 * ESZ) : row_rsrc(logits, 0u), extra_off(gn));
  }
}

int cu_count_of_current_device(int* n_out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return check_launch("hipGetDevice");
  static int cu_count[64] = {0};
  if (dev < 0 || dev >= 64) dev = 0;
  if (cu_count[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cu_count[dev] = n;
  }
  *n_out = cu_count[dev];
  return RRL_OK;
}

// Variants by slab count; a row needs ceil(nvec / 1024) slabs.
template <class Tag, bool EXTRAS>
int launch_resident(const RowArgs& a, int32_t nvec, hipStream_t stream) {
  const int need = (nvec + RNT - 1) / RNT;
  int cus = 0;
  if (int rc = cu_count_of_current_device(&cus)) return rc;
  const int64_t rows = a.B * a.T;
  const unsigned pgrid = (unsigned)((rows + 255) / 256 < 65536 ? (rows + 255) / 256 : 65536);
  hipLaunchKernelGGL(pack_records_kernel, dim3(pgrid), dim3(256), 0, stream, a);
  if (int rc = check_launch("pack_records_kernel")) return rc;
  const unsigned grid = (unsigned)(rows < cus ? rows : cus);
#define RRL_RESIDENT_CASE(SLV)                                                                \
  if (need <= SLV) {                                                                          \
    hipLaunchKernelGGL((resident_fused_kernel<Tag, SLV, EXTRAS>), dim3(grid), dim3(RNT), 0,   \
                       stream, a, nvec);                                                     \
    return check_launch("resident_fused_kernel");                                             \
  }
  RRL_RESIDENT_CASE(4)
  RRL_RESIDENT_CASE(8)
  RRL_RESIDENT_CASE(12)
  RRL_RESIDENT_CASE(16)
  RRL_RESIDENT_CASE(20)
#undef RRL_RESIDENT_CASE
  set_error("resident_fused_kernel: row too long");
  return RRL_EINVAL;
}

template <class Tag, bool EXTRAS>
int launch_resident_bwd(const RowArgs& a, int32_t nvec, hipStream_t stream) {
  const int need = (nvec + RNT - 1) / RNT;
  int cus = 0;
  if (int rc = cu_count_of_current_device(&cus)) return rc;
  const int64_t rows = a.B * a.T;
  const unsigned grid = (unsigned)(rows < cus ? rows : cus);
#define RRL_RESIDENT_CASE(SLV)                                                                \
  if (need <= SLV) {                                                                          \
    hipLaunchKernelGGL((resident_bwd_kernel<Tag, SLV, EXTRAS>), dim3(grid), dim3(RNT), 0,     \
                       stream, a, nvec);                                                     \
    return check_launch("resident_bwd_kernel");                                               \
  }
  RRL_RESIDENT_CASE(4)
  RRL_RESIDENT_CASE(8)
  RRL_RESIDENT_CASE(12)
  RRL_RESIDENT_CASE(16)
  RRL_RESIDENT_CASE(20)
#undef RRL_RESIDENT_CASE
  set_error("resident_bwd_kernel: row too long");
  return RRL_EINVAL;
}

template <class Tag>
int dispatch_resident(int mode, bool extras, const RowArgs& a, int32_t nvec, hipStream_t st) {
  if (mode == 1)
    return extras ? launch_resident_bwd<Tag, true>(a, nvec, st)
                  : launch_resident_bwd<Tag, false>(a, nvec, st);
  return extras ? launch_resident<Tag, true>(a, nvec, st) : launch_resident<Tag, false>(a, nvec, st);
}

constexpr int64_t kMaxResidentVec = 20 * RNT;  // SL = 20 fits 128 VGPRs without spills

}  // namespace

// Takes the register-resident kernel (mode 2: the fused single pass; mode 1:
// rrl_logprob_bwd with the forward's log-probs given) for 16-bit and float32
// logits when the row's 16-byte vectors fit the register budget (V <= 163840
// 16-bit or 81920 float32 entries).  Rows that are 128-byte aligned with
// V % (16 / element size) == 0 take the plain variant.  Other rows take the
// variant with head and tail elements, whose body starts on a 128-byte
// boundary, provided every dlogits row sits at its logits row's offset from a
// 128-byte boundary (same strides mod 128 bytes, as for contiguous tensors or
// in place); failing that, 16-byte aligned rows take the plain variant.
// Otherwise *launched stays false and the caller runs the generic row kernel.
int maybe_launch_resident(const RowArgs& a, int mode, int logits_dtype, hipStream_t stream,
                          bool* launched) {
  *launched = false;
  if (mode == 2 && (a.pp.flags & RRL_POLICY_GENERIC)) return RRL_OK;
  if (mode != 1 && mode != 2) return RRL_OK;
  if (logits_dtype != RRL_BF16 && logits_dtype != RRL_F16 && logits_dtype != RRL_F32)
    return RRL_OK;
  if (a.dl_dt != logits_dtype || a.accumulate) return RRL_OK;
  const int64_t esz = logits_dtype == RRL_F32 ? 4 : 2;
  const int64_t epv = 16 / esz;
  if (a.B * a.T == 0 || a.V / epv > kMaxResidentVec) return RRL_OK;
  if (a.B * a.T >= ((int64_t)1 << 31) || a.T >= ((int64_t)1 << 31)) return RRL_OK;
  const auto al = [&](int64_t elems, int64_t n) { return ((elems * esz) % n) == 0; };
  const auto rows_aligned = [&](int64_t n) {
    return a.V % epv == 0 && (uintptr_t)a.logits % n == 0 && (uintptr_t)a.dl % n == 0 &&
           al(a.ls_b, n) && al(a.ls_t, n) && al(a.ds_b, n) && al(a.ds_t, n);
  };
  const bool same_offset = ((uintptr_t)a.dl - (uintptr_t)a.logits) % kBodyAlign == 0 &&
                           al(a.ds_b - a.ls_b, kBodyAlign) && al(a.ds_t - a.ls_t, kBodyAlign);
  // Plain: 128-byte aligned rows, or 16-byte aligned ones the head/tail
  // variant cannot take.
  const bool aligned = rows_aligned(kBodyAlign) || (!same_offset && rows_aligned(16));
  if (!aligned && !same_offset) return RRL_OK;
  const int32_t nvec = (int32_t)(a.V / epv);
  if (mode == 1) {
    // Scalar loads need 4-byte aligned operands.
    if (a.logp_in == nullptr || a.tgt.ptr == nullptr) return RRL_OK;
    if (((uintptr_t)a.lse | (uintptr_t)a.g | (uintptr_t)a.logp_in) % 4) return RRL_OK;
    if ((uintptr_t)a.tgt.ptr % (a.tgt.dt == RRL_I32 ? 4 : 8)) return RRL_OK;
  } else {
    if (a.logp_dt != RRL_F32 || a.records == nullptr) return RRL_OK;
    if ((uintptr_t)a.records % 16) return RRL_OK;
  }
  *launched = true;
  switch (logits_dtype) {
    case RRL_BF16: return dispatch_resident<TagBF16>(mode, !aligned, a, nvec, stream);
    case RRL_F16: return dispatch_resident<TagF16>(mode, !aligned, a, nvec, stream);
    default: return dispatch_resident<TagF32>(mode, !aligned, a, nvec, stream);
  }
}

}  // namespace rrl
