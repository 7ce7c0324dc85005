// Next-token sampling with behaviour log-probs: the rollout side of the
// RoseRLHF path.  The reference samples in roseinfer/engine.py:1103-1171
// (temperature, top-k, top-p, multinomial over softmax(...).clamp_min(1e-9))
// and never returns the sampled token's log-probability, which
// roserlhf/trajectory.py:15,27-28 requires for every token.  One workgroup
// per row picks the token and forms both log-probabilities in the same launch.
//
// Row layout: slab k, lane j holds elements (k*1024 + j)*VEC .. +VEC-1 (VEC =
// 16 bytes of logits), so every pass streams the row with coalesced 16-byte
// loads, and vocabulary order is (slab, lane, element).  A row is re-read per
// pass (from L2 / the memory-side cache: a 151936-entry bf16 row is 297 KB).
//
// Passes (top-k, top-p and the tie searches only when active):
//   1. row max and its lowest index (greedy choice), NaN/+inf check;
//   2. top-k: radix select of the k-th largest key, 8 bits per pass;
//   3. Z = sum over the candidates of exp(x/T - max);
//   4. top-p: radix select over fixed-point probability mass (exact,
//      order-independent integer sums), descending key order;
//   5. inverse CDF in vocabulary order: per-slab totals, then a lane scan
//      inside the chosen slab;
//   6. log-sum-exp over the other columns and the token's log-prob, in the
//      form the training row kernels use (finish_row).
// Ties at a top-k or top-p threshold are kept lowest index first; they are
// located with the same vocabulary-order search over 0/1 weights.
#include "row_common.hpp"

namespace rrl {

// Philox4x32-10 (J. Salmon, M. Moraes, R. Dror, D. Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011): ten rounds of two 32x32->64
// multiplies with the published multipliers and Weyl key increments.
__host__ __device__ inline void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
  const uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;
  const uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)kM0 * c[0];
    const uint64_t p1 = (uint64_t)kM1 * c[2];
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n1 = (uint32_t)p1;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    const uint32_t n3 = (uint32_t)p0;
    c[0] = n0; c[1] = n1; c[2] = n2; c[3] = n3;
    k0 += kW0;
    k1 += kW1;
  }
}

namespace {

constexpr int SNT = 1024;
constexpr int SWAVES = SNT / 64;
constexpr int MAX_SLABS = 64;
constexpr double kMassScale = 4503599627370496.0;  // 2^52: fixed-point probability

struct SampleArgs {
  const void* logits;
  int64_t B, V, stride;
  float temp;       // 1 when greedy
  int64_t top_k;    // active iff 0 < top_k < V
  double top_p;     // active iff 0 < top_p < 1
  int greedy;
  uint64_t seed, offset;
  int64_t* token;
  float* logp;
  float* logq;
  int32_t* status;
};

// Order-preserving unsigned key of a float's bit pattern (16- or 32-bit).
template <int KB>
__device__ __forceinline__ uint32_t float_key(uint32_t b) {
  constexpr uint32_t sign = 1u << (KB - 1);
  constexpr uint32_t all = KB == 32 ? 0xffffffffu : ((1u << KB) - 1u);
  return (b & sign) ? (~b & all) : (b | sign);
}

template <class Tag> struct Bits;
template <> struct Bits<TagBF16> {
  static constexpr int KB = 16;
  static __device__ __forceinline__ float val(uint32_t u) { return __uint_as_float(u << 16); }
};
template <> struct Bits<TagF16> {
  static constexpr int KB = 16;
  static __device__ __forceinline__ float val(uint32_t u) { return f16_bits_to_f32((uint16_t)u); }
};
template <> struct Bits<TagF32> {
  static constexpr int KB = 32;
  static __device__ __forceinline__ float val(uint32_t u) { return __uint_as_float(u); }
};

// The raw bits of lane `tid`'s elements of slab k (0 past the row's end).
template <class Tag>
__device__ __forceinline__ void load_bits(const typename Tag::S* row, int64_t V, bool al16, int k,
                                          int tid, uint32_t (&u)[Tag::VEC]) {
  constexpr int VEC = Tag::VEC;
  const int64_t e0 = ((int64_t)k * SNT + tid) * VEC;
  if (al16 && e0 + VEC <= V) {
    const uint4 w = *reinterpret_cast<const uint4*>(row + e0);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    if (VEC == 8) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) u[i] = (ws[i >> 1] >> (16 * (i & 1))) & 0xffffu;
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) u[i] = ws[i & 3];
    }
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      uint32_t b = 0;
      if (e0 + i < V) {
        if (sizeof(typename Tag::S) == 2)
          b = reinterpret_cast<const uint16_t*>(row)[e0 + i];
        else
          b = reinterpret_cast<const uint32_t*>(row)[e0 + i];
      }
      u[i] = b;
    }
  }
}

// Raw bits of element e of a row.
template <class Tag>
__device__ __forceinline__ uint32_t load_one(const typename Tag::S* row, long long e) {
  if (sizeof(typename Tag::S) == 2) return reinterpret_cast<const uint16_t*>(row)[e];
  return reinterpret_cast<const uint32_t*>(row)[e];
}

struct SearchShared {
  double wave_slab[SWAVES][MAX_SLABS];
  double slab_tot[MAX_SLABS];
  double wave_tot[SWAVES];
  int wave_i[SWAVES];
  long long wave_l[SWAVES];
  long long sel;
  int last_lane;
};

// Lowest-index maximum over the workgroup: (value, index) pairs, NaN never wins.
__device__ __forceinline__ void argmax_merge(float& bx, long long& bi, float ox, long long oi) {
  if (ox > bx || (ox == bx && oi < bi)) {
    bx = ox;
    bi = oi;
  }
}

// First element, in vocabulary order, whose inclusive prefix of the weights
// exceeds target(total of the weights).  w(e, bits) >= 0 (float) must be a pure
// function of its arguments (it is evaluated twice per element); the prefix
// sums run in float64, so ~1e5 floor weights of 1e-9 next to a weight near 1
// keep their share of the total.  When
// rounding leaves the target at or past the last partial sum, the last
// element with a positive weight is returned; -1 when every weight is 0.
template <class Tag, class WFn, class TFn>
__device__ long long vocab_search(const typename Tag::S* row, int64_t V, bool al16, int nslab,
                                  WFn wfn, TFn tfn, SearchShared& sh) {
  constexpr int VEC = Tag::VEC;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  long long last_pos = -1;
  for (int k = 0; k < nslab; ++k) {
    uint32_t u[VEC];
    load_bits<Tag>(row, V, al16, k, tid, u);
    const long long e0 = ((long long)k * SNT + tid) * VEC;
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float wi = (e0 + i < V) ? wfn(e0 + i, u[i]) : 0.0f;
      asm volatile("" : "+v"(wi));  // the same rounding in both evaluations
      if (wi > 0.0f) last_pos = e0 + i;
      acc += (double)wi;
    }
    acc = wave_sum(acc);
    if (lane == 0) sh.wave_slab[wave][k] = acc;
  }
  // last positive element over the workgroup
  for (int o = 32; o > 0; o >>= 1) {
    const long long t = __shfl_xor(last_pos, o, 64);
    last_pos = t > last_pos ? t : last_pos;
  }
  if (lane == 0) sh.wave_l[wave] = last_pos;
  __syncthreads();
  if (tid < nslab) {
    double s = 0.0;
    for (int w = 0; w < SWAVES; ++w) s += sh.wave_slab[w][tid];
    sh.slab_tot[tid] = s;
  }
  last_pos = sh.wave_l[0];
  for (int w = 1; w < SWAVES; ++w) last_pos = sh.wave_l[w] > last_pos ? sh.wave_l[w] : last_pos;
  __syncthreads();
  double total = 0.0;
  for (int k = 0; k < nslab; ++k) total += sh.slab_tot[k];
  const double target = tfn(total);
  int ks = -1;
  double run = 0.0;
  for (int k = 0; k < nslab; ++k) {
    const double t = sh.slab_tot[k];
    if (t > 0.0 && run + t > target) {
      ks = k;
      break;
    }
    run += t;
  }
  if (ks < 0) return last_pos;  // uniform over the workgroup

  // Lane scan inside slab ks.
  uint32_t u[VEC];
  load_bits<Tag>(row, V, al16, ks, tid, u);
  const long long e0 = ((long long)ks * SNT + tid) * VEC;
  float w8[VEC];
  double lw = 0.0;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    float wi = (e0 + i < V) ? wfn(e0 + i, u[i]) : 0.0f;
    asm volatile("" : "+v"(wi));
    w8[i] = wi;
    lw += (double)wi;
  }
  double incl = lw;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  // Exclusive prefix = the previous lane's inclusive value itself, so that
  // consecutive lanes' [exclusive, inclusive) ranges tile without a gap.
  double excl = __shfl_up(incl, 1, 64);
  if (lane == 0) excl = 0.0;
  int lastl = lw > 0.0 ? tid : -1;
  for (int o = 32; o > 0; o >>= 1) {
    const int t = __shfl_xor(lastl, o, 64);
    lastl = t > lastl ? t : lastl;
  }
  if (lane == 63) sh.wave_tot[wave] = incl;
  if (lane == 0) sh.wave_i[wave] = lastl;
  if (tid == 0) sh.sel = last_pos;  // defined even if no lane claims
  __syncthreads();
  double wpre = run;
  for (int w = 0; w < wave; ++w) wpre += sh.wave_tot[w];
  int last_lane = sh.wave_i[0];
  for (int w = 1; w < SWAVES; ++w) last_lane = sh.wave_i[w] > last_lane ? sh.wave_i[w] : last_lane;
  const double lincl = wpre + incl;
  const double lexcl = wpre + excl;
  // [lexcl, lincl) of consecutive lanes tile the slab's range from `run`
  // (<= target); the last positive lane takes what rounding leaves past the
  // end.
  const bool claim = lw > 0.0 && lexcl <= target && (target < lincl || tid == last_lane);
  if (claim) {
    double cum = lexcl;
    long long pick = -1, lastp = -1;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      if (w8[i] > 0.0f) {
        lastp = e0 + i;
        if (pick < 0 && cum + (double)w8[i] > target) pick = e0 + i;
      }
      cum += (double)w8[i];
    }
    sh.sel = pick >= 0 ? pick : lastp;
  }
  __syncthreads();
  const long long sel = sh.sel;
  __syncthreads();
  return sel;
}

template <class Tag>
__global__ __launch_bounds__(SNT) void sample_kernel(SampleArgs a) {
  using S = typename Tag::S;
  constexpr int VEC = Tag::VEC;
  constexpr int KB = Bits<Tag>::KB;
  __shared__ SearchShared sh;
  __shared__ uint32_t hist[256];
  __shared__ unsigned long long histm[256];
  __shared__ float sh_m[SWAVES], sh_s[SWAVES];
  __shared__ float sh_x[SWAVES];
  __shared__ long long sh_e[SWAVES];
  __shared__ int sh_bad;
  __shared__ uint32_t sh_digit;
  __shared__ int sh_found;
  __shared__ unsigned long long sh_above;

  const int64_t r = blockIdx.x;
  if (r >= a.B) return;
  const S* row = static_cast<const S*>(a.logits) + r * a.stride;
  const int64_t V = a.V;
  const bool al16 = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
  const int nslab = (int)((V + (int64_t)SNT * VEC - 1) / ((int64_t)SNT * VEC));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float T = a.temp;

  // 1. row max with its lowest index; NaN / +inf check.
  float bx = -__builtin_huge_valf();
  long long bi = 0x7fffffffffffffffLL;
  bool bad = false;
  for (int k = 0; k < nslab; ++k) {
    uint32_t u[VEC];
    load_bits<Tag>(row, V, al16, k, tid, u);
    const long long e0 = ((long long)k * SNT + tid) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      if (e0 + i < V) {
        const float x = Bits<Tag>::val(u[i]);
        bad |= (x != x) || (x == __builtin_huge_valf());
        argmax_merge(bx, bi, x, e0 + i);
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ox = __shfl_xor(bx, o, 64);
    const long long oi = __shfl_xor(bi, o, 64);
    argmax_merge(bx, bi, ox, oi);
  }
  if (tid == 0) sh_bad = 0;
  __syncthreads();
  if (bad) sh_bad = 1;
  if (lane == 0) {
    sh_x[wave] = bx;
    sh_e[wave] = bi;
  }
  __syncthreads();
  bx = sh_x[0];
  bi = sh_e[0];
  for (int w = 1; w < SWAVES; ++w) argmax_merge(bx, bi, sh_x[w], sh_e[w]);
  const bool row_bad = sh_bad != 0 || bx == -__builtin_huge_valf();
  __syncthreads();
  if (row_bad) {
    if (tid == 0) {
      raise_flag(a.status, RRL_FLAG_BAD_PROBS);
      a.token[r] = bi < V ? bi : 0;
      a.logp[r] = __builtin_nanf("");
      if (a.logq) a.logq[r] = __builtin_nanf("");
    }
    return;
  }
  const float m = bx / T;  // max of x / T (division by T > 0 is monotone)

  long long tok = bi;
  float logq = 0.0f;
  if (!a.greedy) {
    // 2. top-k candidates: the k-th largest key by an MSB-first radix select.
    const bool use_k = a.top_k > 0 && a.top_k < V;
    uint32_t kth = 0;
    int need_k = 0, cnt_k = 0;
    long long cut_k = -1;
    if (use_k) {
      uint32_t prefix = 0, pmask = 0;
      int kk = (int)a.top_k;
      for (int shift = KB - 8; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += SNT) hist[i] = 0;
        __syncthreads();
        for (int k = 0; k < nslab; ++k) {
          uint32_t u[VEC];
          load_bits<Tag>(row, V, al16, k, tid, u);
          const long long e0 = ((long long)k * SNT + tid) * VEC;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const uint32_t key = float_key<KB>(u[i]);
            if (e0 + i < V && (key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
          }
        }
        __syncthreads();
        if (wave == 0) {
          // lane l owns bins 4l..4l+3; counts above a bin = suffix sums.
          uint32_t c[4];
          for (int b = 0; b < 4; ++b) c[b] = hist[4 * lane + b];
          const uint32_t t = c[0] + c[1] + c[2] + c[3];
          uint32_t incl = t;
          for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_down(incl, o, 64);
            if (lane + o < 64) incl += y;
          }
          uint32_t above = incl - t;
          for (int b = 3; b >= 0; --b) {
            if (above < (uint32_t)kk && (uint32_t)kk <= above + c[b]) {
              sh_digit = 4 * lane + b;
              sh_above = above;
            }
            above += c[b];
          }
        }
        __syncthreads();
        const uint32_t d = sh_digit;
        kk -= (int)sh_above;
        prefix |= d << shift;
        pmask |= 255u << shift;
        cnt_k = (int)hist[d];
        __syncthreads();
      }
      kth = prefix;
      need_k = kk;  // 1 <= need_k <= cnt_k tokens at the threshold are kept
      if (need_k < cnt_k) {
        const double nth = (double)(need_k - 1);
        cut_k = vocab_search<Tag>(
            row, V, al16, nslab,
            [&](long long, uint32_t b) { return float_key<KB>(b) == kth ? 1.0f : 0.0f; },
            [&](double) { return nth; }, sh);
      }
    }
    auto cand = [&](long long e, uint32_t key) {
      return !use_k || key > kth || (key == kth && (need_k >= cnt_k || e <= cut_k));
    };

    // 3. Z over the candidates.
    float zs = 0.0f;
    for (int k = 0; k < nslab; ++k) {
      uint32_t u[VEC];
      load_bits<Tag>(row, V, al16, k, tid, u);
      const long long e0 = ((long long)k * SNT + tid) * VEC;
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        if (e0 + i < V && cand(e0 + i, float_key<KB>(u[i])))
          zs += expf(Bits<Tag>::val(u[i]) / T - m);
      }
    }
    {
      float v1[1] = {zs};
      block_sum<SNT, 1, float>(v1, sh_s);
      zs = v1[0];
    }
    const float inv_z = 1.0f / zs;
    auto prob = [&](uint32_t b) {
      float e = expf(Bits<Tag>::val(b) / T - m);
      asm volatile("" : "+v"(e));
      return e * inv_z;
    };

    // 4. top-p: radix select over fixed-point mass in descending key order.
    const bool use_p = a.top_p > 0.0 && a.top_p < 1.0;
    bool p_found = false;
    uint32_t pth = 0;
    unsigned long long n_keep = 0, cnt_p = 0;
    long long cut_p = -1;
    if (use_p) {
      const unsigned long long P = (unsigned long long)(a.top_p * kMassScale);
      uint32_t prefix = 0, pmask = 0;
      unsigned long long A = 0;
      p_found = true;
      for (int shift = KB - 8; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += SNT) {
          hist[i] = 0;
          histm[i] = 0;
        }
        if (tid == 0) sh_found = 0;
        __syncthreads();
        for (int k = 0; k < nslab; ++k) {
          uint32_t u[VEC];
          load_bits<Tag>(row, V, al16, k, tid, u);
          const long long e0 = ((long long)k * SNT + tid) * VEC;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const uint32_t key = float_key<KB>(u[i]);
            if (e0 + i < V && (key & pmask) == prefix && cand(e0 + i, key)) {
              const unsigned long long fx =
                  (unsigned long long)((double)prob(u[i]) * kMassScale);
              atomicAdd(&hist[(key >> shift) & 255u], 1u);
              atomicAdd(&histm[(key >> shift) & 255u], fx);
            }
          }
        }
        __syncthreads();
        if (wave == 0) {
          unsigned long long c[4];
          for (int b = 0; b < 4; ++b) c[b] = histm[4 * lane + b];
          const unsigned long long t = c[0] + c[1] + c[2] + c[3];
          unsigned long long incl = t;
          for (int o = 1; o < 64; o <<= 1) {
            const unsigned long long y = __shfl_down(incl, o, 64);
            if (lane + o < 64) incl += y;
          }
          unsigned long long above = A + (incl - t);
          for (int b = 3; b >= 0; --b) {
            // the bin holding the first token whose inclusive mass passes P
            if (c[b] > 0 && above <= P && P < above + c[b]) {
              sh_digit = 4 * lane + b;
              sh_above = above;
              sh_found = 1;
            }
            above += c[b];
          }
        }
        __syncthreads();
        const bool f = sh_found != 0;
        const uint32_t d = sh_digit;
        const unsigned long long ab = sh_above;
        const unsigned long long binm = histm[d], binc = hist[d];
        __syncthreads();
        if (!f) {  // every candidate fits under top_p
          p_found = false;
          break;
        }
        A = ab;
        prefix |= d << shift;
        pmask |= 255u << shift;
        cnt_p = binc;
        if (shift == 0 || KB == 8) {
          const unsigned long long each = binm / binc;  // equal keys, equal mass
          n_keep = each > 0 ? (P - A) / each : binc;
        }
      }
      if (p_found) {
        pth = prefix;
        // The first token in descending order (the row maximum) is always kept.
        if (pth == float_key<KB>(load_one<Tag>(row, bi)) && n_keep == 0) n_keep = 1;
        if (n_keep > 0 && n_keep < cnt_p) {
          const double nth = (double)(n_keep - 1);
          cut_p = vocab_search<Tag>(
              row, V, al16, nslab,
              [&](long long e, uint32_t b) {
                const uint32_t key = float_key<KB>(b);
                return (key == pth && cand(e, key)) ? 1.0f : 0.0f;
              },
              [&](double) { return nth; }, sh);
        }
      }
    }
    auto kept = [&](long long e, uint32_t key) {
      return !p_found || key > pth ||
             (key == pth && (n_keep >= cnt_p || (n_keep > 0 && e <= cut_p)));
    };
    auto qw = [&](long long e, uint32_t b) {
      const uint32_t key = float_key<KB>(b);
      if (!cand(e, key)) return 0.0f;
      const float p = kept(e, key) ? prob(b) : 0.0f;
      return fmaxf(p, 1e-9f);
    };

    // 5. inverse CDF with this row's uniform.
    uint32_t c[4] = {(uint32_t)r, (uint32_t)((uint64_t)r >> 32), (uint32_t)a.offset,
                     (uint32_t)(a.offset >> 32)};
    philox4x32_10(c, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
    const double u01 = (double)(c[0] >> 8) * 5.9604644775390625e-8;  // 2^-24
    __shared__ double sh_total;
    tok = vocab_search<Tag>(
        row, V, al16, nslab, qw,
        [&](double total) {
          if (tid == 0) sh_total = total;
          return u01 * total;
        },
        sh);
    __syncthreads();
    const double qtot = sh_total;
    if (tok < 0 || tok >= V) tok = bi;  // no positive weight: cannot happen, q >= 1e-9
    if (tid == 0) logq = (float)(log((double)qw(tok, load_one<Tag>(row, tok))) - log(qtot));
  }

  // 6. log_softmax(x / T) at the token, as the training row kernels form it.
  const float xt = Bits<Tag>::val(load_one<Tag>(row, tok)) / T;
  float mm = -__builtin_huge_valf(), ss = 0.0f;
  for (int k = 0; k < nslab; ++k) {
    uint32_t u[VEC];
    load_bits<Tag>(row, V, al16, k, tid, u);
    const long long e0 = ((long long)k * SNT + tid) * VEC;
    float v[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i)
      v[i] = e0 + i < V ? Bits<Tag>::val(u[i]) / T : -__builtin_huge_valf();
    const long long rel = tok - e0;
    online_update<float, VEC>(mm, ss, v, (rel >= 0 && rel < VEC) ? (int)rel : -1);
  }
  block_online_combine<SNT, float>(mm, ss, sh_m, sh_s);
  if (tid == 0) {
    const RowLogprob<float> fr = finish_row<float>(mm, ss, xt);
    a.token[r] = tok;
    a.logp[r] = fr.logp;
    if (a.logq) a.logq[r] = logq;
  }
}

template <class Tag>
int launch_sample(const SampleArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((sample_kernel<Tag>), dim3((unsigned)a.B), dim3(SNT), 0, st, a);
  return check_launch("sample_kernel");
}

}  // namespace
}  // namespace rrl

using namespace rrl;

extern "C" void rrl_philox4x32_10(uint32_t ctr[4], const uint32_t key[2]) {
  uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
  philox4x32_10(c, key[0], key[1]);
  for (int i = 0; i < 4; ++i) ctr[i] = c[i];
}

extern "C" int rrl_sample_logprobs(const void* logits, int32_t logits_dtype, int64_t B, int64_t V,
                                   int64_t row_stride, double temperature, int64_t top_k,
                                   double top_p, int32_t do_sample, uint64_t seed,
                                   uint64_t offset, int64_t* token_out, float* logp_out,
                                   float* logq_out, int32_t* status, void* stream) {
  clear_error();
  RRL_REQUIRE(logits_dtype == RRL_F32 || logits_dtype == RRL_BF16 || logits_dtype == RRL_F16,
              RRL_EDTYPE, "sampling logits must be float32, bfloat16 or float16");
  RRL_REQUIRE(B >= 0 && V >= 1, RRL_EINVAL, "sampling needs B >= 0 rows of V >= 1 logits");
  if (B == 0) return RRL_OK;
  const int vec = logits_dtype == RRL_F32 ? 4 : 8;
  RRL_REQUIRE(V <= (int64_t)SNT * vec * MAX_SLABS, RRL_EINVAL, "vocabulary too large for the sampler");
  RRL_REQUIRE(B < (1LL << 31), RRL_EINVAL, "too many rows");
  RRL_REQUIRE(logits && token_out && logp_out, RRL_EINVAL, "null pointer argument");
  RRL_REQUIRE(((uintptr_t)logits % dtype_size(logits_dtype)) == 0, RRL_EALIGN,
              "logits pointer misaligned");
  const bool greedy = do_sample == 0 || !(temperature > 0.0);
  SampleArgs a{};
  a.logits = logits; a.B = B; a.V = V; a.stride = row_stride;
  a.temp = greedy ? 1.0f : (float)temperature;
  RRL_REQUIRE(greedy || a.temp > 0.0f, RRL_EINVAL, "temperature underflows float32");
  a.top_k = top_k; a.top_p = top_p; a.greedy = greedy ? 1 : 0;
  a.seed = seed; a.offset = offset;
  a.token = token_out; a.logp = logp_out; a.logq = logq_out; a.status = status;
  hipStream_t st = as_stream(stream);
  switch (logits_dtype) {
    case RRL_BF16: return launch_sample<TagBF16>(a, st);
    case RRL_F16: return launch_sample<TagF16>(a, st);
    default: return launch_sample<TagF32>(a, st);
  }
}
