// Next-token sampling with behaviour log-probs: the rollout side of the
// RoseRLHF path.  The reference samples in roseinfer/engine.py:1103-1171
// (temperature, top-k, top-p, multinomial over softmax(...).clamp_min(1e-9))
// and never returns the sampled token's log-probability, which
// roserlhf/trajectory.py:15,27-28 requires for every token.  One workgroup
// per row picks the token and forms both log-probabilities in the same launch.
//
// Row layout: slab k, lane j holds elements (k*1024 + j)*VEC .. +VEC-1 (VEC =
// 16 bytes of logits), so every pass moves the row with coalesced 16-byte
// loads, and vocabulary order is (slab, lane, element).  Three kernels:
//   * sample_blocks_kernel (plain sampling, greedy decoding, and top-p
//     without top-k on bfloat16 rows) and
//     sample_resident_kernel (top-k with or without top-p), both for 16-bit
//     rows made of whole, aligned 16-byte vectors: the row stays in VGPRs
//     and is read from memory once; their sweeps are described at their
//     definitions.
//   * sample_kernel (everything else): a row is re-read per pass (from L2 /
//     the memory-side cache: a 151936-entry bf16 row is 297 KB).
// Without top-k / top-p, max(p, 1e-9) is drawn as the mixture of p
// (probability 1 / (1 + G)) and the floor's excess max(1e-9 - p, 0)
// (probability G / (1 + G), G its total), a second uniform choosing the
// component: (1 / (1 + G)) p + (G / (1 + G)) (g / G) = max(p, 1e-9) / (1 + G).
//
// sample_kernel's passes (top-k, top-p and the tie searches only when active):
//   1. row max and its lowest index (greedy choice), the sums of
//      exp((x - max)/T) over every entry (Z without top-k) and over every
//      entry but the maximum (the greedy token's S_other), NaN/+inf check;
//   2. top-k: radix select of the k-th largest key, 8 bits per pass;
//   3. Z = sum over the candidates of exp(x/T - max);
//   4. top-p: radix select over fixed-point probability mass (exact,
//      order-independent integer sums), descending key order;
//   5. inverse CDF in vocabulary order (of the chosen mixture component
//      without top-k / top-p): per-slab totals, then a lane scan inside the
//      chosen slab;
//   6. the token's log-prob in the form the training row kernels use
//      (finish_row), from pass 1's sums.
// Greedy decoding is pass 1 alone; sampling without top-k / top-p is passes 1
// and 5.  With top-k (k <= 1024), one pass after step 2 gathers the entries
// at or above the k-th key into LDS and steps 3-5 run on that list, one
// candidate per thread, without re-reading the row.
// Ties at a top-k or top-p threshold are kept lowest index first; they are
// located with the same vocabulary-order search over 0/1 weights.
#include "row_common.hpp"
#include "wave_common.hpp"

#include <type_traits>

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
  int fill_in;  // sample_kernel: only the rows whose token slot holds -1
};

// Order-preserving unsigned key of a float's bit pattern (16- or 32-bit).
// -0 takes +0's key: the two compare equal, so at a top-k or top-p threshold
// they are one group of ties, kept lowest index first (as value comparisons
// rank them).
template <int KB>
__device__ __forceinline__ uint32_t float_key(uint32_t b) {
  constexpr uint32_t sign = 1u << (KB - 1);
  constexpr uint32_t all = KB == 32 ? 0xffffffffu : ((1u << KB) - 1u);
  b = (b & (all ^ sign)) == 0u ? 0u : b;
  return (b & sign) ? (~b & all) : (b | sign);
}

// The bit pattern whose float_key is `key`.
template <int KB>
__device__ __forceinline__ uint32_t key_bits(uint32_t key) {
  constexpr uint32_t sign = 1u << (KB - 1);
  constexpr uint32_t all = KB == 32 ? 0xffffffffu : ((1u << KB) - 1u);
  return (key & sign) ? (key & ~sign) : (~key & all);
}

template <class Tag> struct Bits;
template <> struct Bits<TagBF16> {
  static constexpr uint32_t NEG_INF = 0xFF80FF80u;  // -inf in every element of a dword
  static constexpr int KB = 16;
  static __device__ __forceinline__ float val(uint32_t u) { return __uint_as_float(u << 16); }
  static __device__ __forceinline__ uint32_t bits_of(float v) { return __float_as_uint(v) >> 16; }
};
template <> struct Bits<TagF16> {
  static constexpr uint32_t NEG_INF = 0xFC00FC00u;  // -inf in every element of a dword
  static constexpr int KB = 16;
  static __device__ __forceinline__ float val(uint32_t u) { return f16_bits_to_f32((uint16_t)u); }
  static __device__ __forceinline__ uint32_t bits_of(float v) { return f32_to_f16_bits(v); }
};
template <> struct Bits<TagF32> {
  static constexpr uint32_t NEG_INF = 0xFF800000u;  // -inf in every element of a dword
  static constexpr int KB = 32;
  static __device__ __forceinline__ float val(uint32_t u) { return __uint_as_float(u); }
  static __device__ __forceinline__ uint32_t bits_of(float v) { return __float_as_uint(v); }
};

// Lane `tid`'s 16 bytes of slab k as stored (zeros past the row's end); a
// row that is not 16-byte aligned, or the row's last partial vector, is read
// element by element.
template <class Tag>
__device__ __forceinline__ uint4 load_raw(const typename Tag::S* row, int V, bool al16, int k,
                                          int tid) {
  constexpr int VEC = Tag::VEC;
  const int e0 = (k * SNT + tid) * VEC;
  if (al16 && e0 + VEC <= V) return *reinterpret_cast<const uint4*>(row + e0);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    if (e0 + i < V) {
      if (VEC == 8)
        w[i >> 1] |= (uint32_t)reinterpret_cast<const uint16_t*>(row)[e0 + i] << (16 * (i & 1));
      else
        w[i] = reinterpret_cast<const uint32_t*>(row)[e0 + i];
    }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

template <class Tag>
__device__ __forceinline__ void unpack_raw(const uint4& v, uint32_t (&u)[Tag::VEC]) {
  const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
  if (Tag::VEC == 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = (ws[i >> 1] >> (16 * (i & 1))) & 0xffffu;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = ws[i];
  }
}

// f(k, e0, u, full) over the slabs of this lane, ten (f16: eight) slab loads
// in flight at a time: a pass re-reads the row from memory, and each batch costs one
// memory latency, so a 19-slab bf16 row of 151936 entries takes two per pass.
// `full` is std::true_type for a slab that lies inside the row in every lane
// (all but the last), so f's per-element bounds checks fold away there; the
// row's last, partial slab gets std::false_type.
template <class Tag, class F>
__device__ __forceinline__ void for_slabs(const typename Tag::S* row, int V, bool al16, int nslab,
                                          F&& f) {
  constexpr int VEC = Tag::VEC;
  // f16's conversions need more registers per slab than bf16 or f32 shifts.
  constexpr int UNR = std::is_same<Tag, TagF16>::value ? 8 : 10;
  const int tid = threadIdx.x;
  const int nfull = V / (SNT * VEC);
  for (int k0 = 0; k0 < nfull; k0 += UNR) {
    uint4 w[UNR];
#pragma unroll
    for (int j = 0; j < UNR; ++j)
      w[j] = (k0 + j < nfull) ? load_raw<Tag>(row, V, al16, k0 + j, tid) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < UNR; ++j) {
      if (k0 + j < nfull) {
        uint32_t u[VEC];
        unpack_raw<Tag>(w[j], u);
        f(k0 + j, ((k0 + j) * SNT + tid) * VEC, u, std::true_type{});
      }
    }
  }
  if (nfull < nslab) {
    uint32_t u[VEC];
    unpack_raw<Tag>(load_raw<Tag>(row, V, al16, nfull, tid), u);
    f(nfull, (nfull * SNT + tid) * VEC, u, std::false_type{});
  }
}

// Wave64 sum, the same value in every lane: DPP butterflies inside each row
// of 16 lanes (quad_perm [1,0,3,2], [2,3,0,1], then the half-row and row
// mirrors), then the four row results through readlane.  VALU-latency steps
// instead of a chain of LDS-permute round trips.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const unsigned long long lo = dpp_u32<CTRL>((uint32_t)b);
  const unsigned long long hi = dpp_u32<CTRL>((uint32_t)(b >> 32));
  return __longlong_as_double((long long)((hi << 32) | lo));
}
__device__ __forceinline__ double lane_read_f64(double v, int l) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const unsigned long long lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
  const unsigned long long hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
  return __longlong_as_double((long long)((hi << 32) | lo));
}
__device__ __forceinline__ double wave_sum_d(double v) {
  v += dpp_f64<0xB1>(v);
  v += dpp_f64<0x4E>(v);
  v += dpp_f64<0x141>(v);
  v += dpp_f64<0x140>(v);
  return (lane_read_f64(v, 0) + lane_read_f64(v, 16)) + (lane_read_f64(v, 32) + lane_read_f64(v, 48));
}

// Raw bits of element e of a row.
template <class Tag>
__device__ __forceinline__ uint32_t load_one(const typename Tag::S* row, int e) {
  if (sizeof(typename Tag::S) == 2) return reinterpret_cast<const uint16_t*>(row)[e];
  return reinterpret_cast<const uint32_t*>(row)[e];
}

struct SearchShared {
  double wave_slab[SWAVES][MAX_SLABS];
  double slab_tot[MAX_SLABS];
  double wave_tot[SWAVES];
  int wave_i[SWAVES];
  int wave_l[SWAVES];
  int sel;
};

// Top-k candidates held in LDS, one per thread (top_k <= KCAP).
constexpr int KCAP = SNT;
// The register-resident top-k gather's tail past KCAP (in LDS a short list's
// draw uses otherwise).
constexpr int OVF = 3 * SNT;
// Keys counted by the register-resident top-p path (16 KB of LDS).
constexpr int TOPP_BINS = 4 * SNT;

struct CandShared {
  int n;                          // entries gathered (may exceed KCAP: then unused)
  int idx[KCAP];                  // vocabulary index: gathered, then dense candidates
  uint32_t bits[KCAP];            // the entry as stored
  int sidx[KCAP];                 // the gathered entries sorted by index
  uint32_t sbits[KCAP];
  unsigned long long mass[KCAP];  // top-p: fixed-point probability of candidate i
  uint32_t key[KCAP];
  int wave_cnt[SWAVES];
  double wave_sum[SWAVES];
  int found;                      // top-p threshold group
  uint32_t pth;
  unsigned long long A, M;
  int C;
  int pick;
  float logq;
};

// Number of threads below this one (in thread order) whose flag is set, and
// the total over the workgroup.
__device__ __forceinline__ int block_excl_count(bool flag, int* wave_cnt, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned long long m = __ballot(flag);
  const int below = __popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) wave_cnt[wave] = __popcll(m);
  __syncthreads();
  int pre = 0, tot = 0;
  for (int w = 0; w < SWAVES; ++w) {
    const int c = wave_cnt[w];
    pre += w < wave ? c : 0;
    tot += c;
  }
  __syncthreads();
  total = tot;
  return pre + below;
}

// Inclusive and exclusive prefix sums of v in thread order and the total.  A
// thread's exclusive value is exactly the previous thread's inclusive one
// (the same operands in the same order), so the [excl, incl) ranges tile.
__device__ __forceinline__ void block_scan_d(double v, double* wave_sum, double& incl,
                                             double& excl, double& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  double in = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double t = __shfl_up(in, o, 64);
    if (lane >= o) in += t;
  }
  const double prev = __shfl_up(in, 1, 64);
  if (lane == 63) wave_sum[wave] = in;
  __syncthreads();
  double pre = 0.0, tot = 0.0;  // one summation order in every thread
  for (int w = 0; w < SWAVES; ++w) {
    if (w == wave) pre = tot;
    tot += wave_sum[w];
  }
  __syncthreads();
  incl = pre + in;
  excl = lane == 0 ? pre : pre + prev;
  total = tot;
}

// Lowest-index maximum over the workgroup: (value, index) pairs, NaN never wins.
__device__ __forceinline__ void argmax_merge(float& bx, int& bi, float ox, int oi) {
  if (ox > bx || (ox == bx && oi < bi)) {
    bx = ox;
    bi = oi;
  }
}

// Minimum of v over the workgroup (every thread takes part; the result is
// the same in every thread).
__device__ __forceinline__ int block_min_i32(int v) {
  __shared__ int sh_min[SWAVES];
  v = wave_min_dpp(v);
  if ((threadIdx.x & 63) == 0) sh_min[threadIdx.x >> 6] = v;
  __syncthreads();
  int m = sh_min[0];
  for (int w = 1; w < SWAVES; ++w) m = min(m, sh_min[w]);
  __syncthreads();
  return m;
}

// First element, in vocabulary order, whose inclusive prefix of the weights
// exceeds target(total of the weights).  wfn(e, bits) >= 0 must be a pure
// function of its arguments (it is evaluated twice per element).  Each lane
// adds its 8 (or 4) weights in float32 and the groups in float64, so ~1e5
// floor weights of 1e-9 next to a weight near 1 keep their share of the
// total.  When rounding leaves the target at or past the last partial sum,
// the last element with a positive weight is returned; -1 when every weight
// is 0.
//
// ALL_POSITIVE: every element's weight is known to be > 0 (the floored
// distribution without top-k / top-p), so the last positive element is V - 1
// and is not tracked per element.
template <class Tag, bool ALL_POSITIVE, class WFn, class TFn>
__device__ __forceinline__ int vocab_search(const typename Tag::S* row, int V, bool al16,
                                                  int nslab, WFn wfn, TFn tfn, SearchShared& sh) {
  constexpr int VEC = Tag::VEC;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int last_pos = -1;
  for_slabs<Tag>(row, V, al16, nslab, [&](int k, int e0, const uint32_t (&u)[VEC], auto full) {
    float facc = 0.0f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float w = 0.0f;
      if (full || e0 + i < V) w = wfn(e0 + i, u[i]);
      asm volatile("" : "+v"(w));  // the same rounding in both evaluations
      if (!ALL_POSITIVE && w > 0.0f) last_pos = e0 + i;
      facc += w;
    }
    const double acc = wave_sum_d((double)facc);
    if (lane == 0) sh.wave_slab[wave][k] = acc;
  });
  // last positive element over the workgroup
  if (ALL_POSITIVE) last_pos = V - 1;
  for (int o = 32; o > 0; o >>= 1) {
    const int t = __shfl_xor(last_pos, o, 64);
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
  unpack_raw<Tag>(load_raw<Tag>(row, V, al16, ks, tid), u);
  const int e0 = (ks * SNT + tid) * VEC;
  float w8[VEC];
  float flw = 0.0f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    float w = 0.0f;
    if (e0 + i < V) w = wfn(e0 + i, u[i]);
    asm volatile("" : "+v"(w));
    w8[i] = w;
    flw += w;
  }
  const double lw = (double)flw;
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
    int pick = -1, lastp = -1;
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
  const int sel = sh.sel;
  __syncthreads();
  return sel;
}

// Top-k (and top-p) draw from a candidate list in LDS, one entry per thread:
// cs.idx / cs.bits hold n <= KCAP entries (vocabulary index, stored bits) in
// any order, among them every entry whose key is >= kth.  The k candidates are
// every entry above the k-th key kth and the first need_k entries at it,
// lowest index first.  Z is taken over the candidates with exp(x/T - m)
// (m = the row maximum of x/T), top-p is the radix select's threshold group
// from exact integer sums over the list (max_key: the key of the row
// maximum, which is always kept), and the token is drawn by inverse CDF over
// the floored q in vocabulary order with the uniform u01.  Every thread
// returns the token, log q(token) and the token's stored bits.
// Top-p's threshold group over a candidate list: the key t (KB-bit order
// key ck of the threads with mine set, fixed-point mass ms) whose group
// holds P, A <= P < A + M, with A the mass of the keys above t and M the
// group's own (the groups' [A, A + M) tile [0, total mass), so at most one
// does).  MSB-first radix select, 8 bits per pass, over 256-bin histograms
// of mass and count (exact integer sums, in any order); cs.mass and cs.key
// serve as the bins.  Returns false when P lies past the total (every
// candidate kept); else cs.pth, cs.A, cs.M and cs.C describe the group.
template <int KB>
__device__ __forceinline__ bool mass_threshold(bool mine, uint32_t ck, unsigned long long ms,
                                               unsigned long long P, CandShared& cs) {
  static_assert(KB == 16 || KB == 32, "16- or 32-bit keys");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  unsigned long long* hm = cs.mass;
  uint32_t* hc = cs.key;
  uint32_t prefix = 0, pmask = 0;
  unsigned long long Pr = P, A = 0;
#pragma unroll
  for (int pass = 0; pass < KB / 8; ++pass) {
    const int shift = KB - 8 - 8 * pass;
    if (tid < 256) {
      hm[tid] = 0ull;
      hc[tid] = 0u;
    }
    if (tid == 0) cs.found = 0;
    __syncthreads();
    if (mine && (ck & pmask) == prefix) {
      const uint32_t d = (ck >> shift) & 255u;
      atomicAdd(&hm[d], ms);
      atomicAdd(&hc[d], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      // lane l owns bins 4l..4l+3; the mass above a bin is a suffix sum.
      unsigned long long c[4];
      for (int b = 0; b < 4; ++b) c[b] = hm[4 * lane + b];
      const unsigned long long t = c[0] + c[1] + c[2] + c[3];
      unsigned long long incl = t;
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long y = __shfl_down(incl, o, 64);
        if (lane + o < 64) incl += y;
      }
      unsigned long long above = incl - t;
      for (int b = 3; b >= 0; --b) {
        if (above <= Pr && Pr - above < c[b]) {
          cs.found = 1;
          cs.pth = 4 * lane + b;
          cs.A = above;
          cs.M = c[b];
          cs.C = (int)hc[4 * lane + b];
        }
        above += c[b];
      }
    }
    __syncthreads();
    const bool found = cs.found != 0;
    const uint32_t d = cs.pth;
    const unsigned long long ab = cs.A;
    __syncthreads();  // the next pass clears what was just read
    if (!found) return false;
    Pr -= ab;
    A += ab;
    prefix |= d << shift;
    pmask |= 255u << shift;
  }
  // cs.M and cs.C are the last pass's bin: the group itself.
  if (tid == 0) {
    cs.pth = prefix;
    cs.A = A;
  }
  __syncthreads();
  return true;
}

template <class Tag>
__device__ __forceinline__ void list_draw(CandShared& cs, float* sh_s, int n, uint32_t kth,
                                          int need_k, bool use_p, double top_p, float iT,
                                          float m, uint32_t max_key, double u01, int& tok,
                                          float& logq, uint32_t& tok_bits, bool sorted = false) {
  constexpr int KB = Bits<Tag>::KB;
  const int tid = threadIdx.x;
  // Sort by vocabulary index into sidx / sbits (unless the caller listed
  // idx / bits in that order): an entry's rank is the number of smaller
  // indices.
  if (!sorted) {
    if (tid < n) {
      const int e = cs.idx[tid];
      int rank = 0;
      for (int j = 0; j < n; ++j) rank += cs.idx[j] < e ? 1 : 0;
      cs.sidx[rank] = e;
      cs.sbits[rank] = cs.bits[tid];
    }
    __syncthreads();
  }
  // The k candidates: every entry above the k-th key and the first need_k
  // entries at it, lowest index first; relaid densely in index order.
  const bool have = tid < n;
  const int se = have ? (sorted ? cs.idx[tid] : cs.sidx[tid]) : 0;
  const uint32_t sb = have ? (sorted ? cs.bits[tid] : cs.sbits[tid]) : 0u;
  const uint32_t skey = float_key<KB>(sb);
  const bool tie = have && skey == kth;
  int ntie = 0;
  const int tie_rank = block_excl_count(tie, cs.wave_cnt, ntie);
  const bool is_cand = have && (skey > kth || (tie && tie_rank < need_k));
  int kc = 0;
  const int pos = block_excl_count(is_cand, cs.wave_cnt, kc);
  if (is_cand) {
    cs.idx[pos] = se;
    cs.bits[pos] = sb;
  }
  __syncthreads();
  const bool mine = tid < kc;
  const uint32_t cb = mine ? cs.bits[tid] : 0u;
  const uint32_t ck = float_key<KB>(cb);
  // Z over the candidates, with the general path's exp(x/T - m).
  const float ev = mine ? expf(Bits<Tag>::val(cb) * iT - m) : 0.0f;
  float zt[1] = {ev};
  block_sum<SNT, 1, float>(zt, sh_s);
  const float pc = ev * (1.0f / zt[0]);
  // Top-p over the candidates: the radix select's threshold group (first
  // key, in descending order, whose inclusive fixed-point mass passes P),
  // from exact integer sums over the list.
  bool keep = true;
  if (use_p) {
    const unsigned long long P = (unsigned long long)(top_p * kMassScale);
    const unsigned long long ms = mine ? (unsigned long long)((double)pc * kMassScale) : 0ull;
    if (mass_threshold<KB>(mine, ck, ms, P, cs)) {
      const uint32_t pth = cs.pth;
      const unsigned long long A0 = cs.A, C0 = (unsigned long long)cs.C;
      const unsigned long long each = cs.M / C0;  // equal keys, equal mass
      int ntie = 0;
      const int tr = block_excl_count(mine && ck == pth, cs.wave_cnt, ntie);  // index order
      unsigned long long n_keep = each > 0 ? (P - A0) / each : C0;
      // The first token in descending order (the row maximum) is always kept.
      if (pth == max_key && n_keep == 0) n_keep = 1;
      keep = ck > pth ||
             (ck == pth && (n_keep >= C0 || (n_keep > 0 && (unsigned long long)tr < n_keep)));
    }
  }
  // Inverse CDF over the candidates in vocabulary order.
  const float wf = mine ? fmaxf(keep ? pc : 0.0f, 1e-9f) : 0.0f;
  double incl, excl, tot;
  block_scan_d((double)wf, cs.wave_sum, incl, excl, tot);
  const double tgt = u01 * tot;
  if (tid == 0) {
    cs.pick = kc - 1;  // rounding past the last sum: the last candidate
    cs.logq = 0.0f;
  }
  __syncthreads();
  if (mine && excl <= tgt && tgt < incl) cs.pick = tid;
  __syncthreads();
  if (tid == cs.pick) cs.logq = (float)(log((double)wf) - log(tot));
  __syncthreads();
  tok = cs.idx[cs.pick];
  tok_bits = cs.bits[cs.pick];
  logq = cs.logq;
  __syncthreads();
}

// One row of the streaming path, by the whole workgroup (every thread calls
// it): sample_kernel's body, and the register-resident top-k kernel's path
// for a row whose candidate list overflows.  cs and hist: the caller's LDS.
template <class Tag>
__device__ __forceinline__ void sample_row(const SampleArgs& a, const int64_t r, CandShared& cs,
                                           uint32_t* hist) {
  using S = typename Tag::S;
  constexpr int VEC = Tag::VEC;
  constexpr int KB = Bits<Tag>::KB;
  __shared__ SearchShared sh;
  __shared__ unsigned long long histm[256];
  __shared__ float sh_s[2 * SWAVES];
  __shared__ float sh_x[SWAVES];
  __shared__ int sh_e[SWAVES];
  __shared__ uint32_t sh_digit;
  __shared__ int sh_found;
  __shared__ unsigned long long sh_above;

  const S* row = static_cast<const S*>(a.logits) + r * a.stride;
  const int V = (int)a.V;  // at most SNT * VEC * MAX_SLABS (checked on the host)
  const bool al16 = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
  const int nslab = (V + SNT * VEC - 1) / (SNT * VEC);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // x / T as x * (1/T): within an ulp of the division, and one multiply in
  // the per-element work (the sampler is bound by its VALU issue rate).
  const float iT = 1.0f / a.temp;

  // 1. Per lane: the first maximum of the logits and its index, and the sum
  // of exp((x - max) / T) over the lane's other entries.  A lane walks its
  // slabs in increasing index order and keeps the first of equal maxima
  // (strict >); fmaxf skips NaN, so NaN never wins, while NaN and +inf reach
  // the sum (2^NaN, 2^(inf - inf)) and are caught there.  The maximum's own
  // term (exactly 1) is kept out of the sum and added back per lane below, so
  // S_other of the greedy token needs no subtraction and no second pass.
  const float c2 = iT * kLog2e;  // exp(y / T) = 2^(y * c2)
  float bx = -__builtin_huge_valf();
  int bi32 = 0x7fffffff;
  float sx = 0.0f;
  for_slabs<Tag>(row, V, al16, nslab, [&](int, int e0, const uint32_t (&u)[VEC], auto full) {
    float v[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i)
      v[i] = (full || e0 + i < V) ? Bits<Tag>::val(u[i]) : -__builtin_huge_valf();
    float mc = v[0];
#pragma unroll
    for (int i = 1; i < VEC; ++i) mc = fmaxf(mc, v[i]);
    int ic = VEC - 1;
#pragma unroll
    for (int i = VEC - 2; i >= 0; --i) ic = (v[i] == mc) ? i : ic;
    const bool up = mc > bx;
    const int skip = up ? ic : -1;  // the new maximum's own term stays out
    const float mn = fmaxf(bx, mc);
    const float mg = fmaxf(mn, -__FLT_MAX__);
    float es = 0.0f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) es += (i == skip) ? 0.0f : exp2_hw((v[i] - mg) * c2);
    // A replaced maximum joins the other entries with its term 1.
    const float old_term = (up && bx > -__builtin_huge_valf()) ? 1.0f : 0.0f;
    sx = __builtin_fmaf(sx + old_term, exp2_hw((bx - mg) * c2), es);
    bi32 = up ? e0 + ic : bi32;
    bx = mn;
  });
  const float lane_max = bx;
  const int lane_arg = bi32;
  int bi = bi32;
  for (int o = 32; o > 0; o >>= 1) {
    const float ox = __shfl_xor(bx, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    argmax_merge(bx, bi, ox, oi);
  }
  if (lane == 0) {
    sh_x[wave] = bx;
    sh_e[wave] = bi;
  }
  __syncthreads();
  bx = sh_x[0];
  bi = sh_e[0];
  for (int w = 1; w < SWAVES; ++w) argmax_merge(bx, bi, sh_x[w], sh_e[w]);
  __syncthreads();
  // Row totals relative to the row maximum: every entry (Z without top-k),
  // and every entry but the argmax (the greedy token's S_other).
  float tot[2];
  {
    const float own = lane_max > -__builtin_huge_valf() ? 1.0f : 0.0f;
    const float f = bx > -__builtin_huge_valf() ? exp2_hw((lane_max - bx) * c2) : 0.0f;
    tot[0] = (sx + own) * f;
    tot[1] = (sx + (lane_arg == bi ? 0.0f : own)) * f;
  }
  block_sum<SNT, 2, float>(tot, sh_s);
  const float os = tot[0], s_arg_other = tot[1];
  const bool row_bad = bx == -__builtin_huge_valf() || bi >= V || os != os ||
                       __builtin_fabsf(bx * iT) == __builtin_huge_valf();
  if (row_bad) {
    int tok_bad = bi < V ? bi : 0;
    if (a.greedy && os != os) {
      // Greedy decoding is torch.argmax, which ranks NaN above every number:
      // the row's first NaN is its token.
      int fn = 0x7fffffff;
      for_slabs<Tag>(row, V, al16, nslab, [&](int, int e0, const uint32_t (&u)[VEC], auto full) {
#pragma unroll
        for (int i = VEC - 1; i >= 0; --i) {
          const float v = Bits<Tag>::val(u[i]);
          if ((full || e0 + i < V) && v != v) fn = min(fn, e0 + i);
        }
      });
      fn = block_min_i32(fn);
      if (fn < V) tok_bad = fn;
    }
    if (tid == 0) {
      raise_flag(a.status, RRL_FLAG_BAD_PROBS);
      a.token[r] = tok_bad;
      a.logp[r] = __builtin_nanf("");
      if (a.logq) a.logq[r] = __builtin_nanf("");
    }
    return;
  }
  const float m = bx * iT;  // max of x / T (scaling by 1/T > 0 is monotone)

  int tok = bi;
  float logq = 0.0f;
  float s_other = s_arg_other;  // the argmax's; replaced below for another token
  if (!a.greedy) {
    // 2. top-k candidates: the k-th largest key by an MSB-first radix select.
    const bool use_k = a.top_k > 0 && a.top_k < V;
    uint32_t kth = 0;
    int need_k = 0, cnt_k = 0;
    int cut_k = -1;
    bool listed = false;  // the top-k candidates sit in LDS (cs), in index order
    if (use_k) {
      uint32_t prefix = 0, pmask = 0;
      int kk = (int)a.top_k;
      for (int shift = KB - 8; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += SNT) hist[i] = 0;
        __syncthreads();
        for_slabs<Tag>(row, V, al16, nslab, [&](int, int e0, const uint32_t (&u)[VEC], auto full) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const uint32_t key = float_key<KB>(u[i]);
            if ((full || e0 + i < V) && (key & pmask) == prefix)
              atomicAdd(&hist[(key >> shift) & 255u], 1u);
          }
        });
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
      // Gather every entry at or above the k-th key (k - need_k + cnt_k of
      // them) into LDS: the rest of the draw then never re-reads the row.
      if (a.top_k <= KCAP) {
        if (tid == 0) cs.n = 0;
        __syncthreads();
        for_slabs<Tag>(row, V, al16, nslab, [&](int, int e0, const uint32_t (&u)[VEC], auto full) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            if ((full || e0 + i < V) && float_key<KB>(u[i]) >= kth) {
              const int p = atomicAdd(&cs.n, 1);
              if (p < KCAP) {
                cs.idx[p] = e0 + i;
                cs.bits[p] = u[i];
              }
            }
          }
        });
        __syncthreads();
        listed = cs.n <= KCAP;
      }
      if (!listed && need_k < cnt_k) {
        const double nth = (double)(need_k - 1);
        cut_k = vocab_search<Tag, false>(
            row, V, al16, nslab,
            [&](int, uint32_t b) { return float_key<KB>(b) == kth ? 1.0f : 0.0f; },
            [&](double) { return nth; }, sh);
      }
    }
    const bool use_p = a.top_p > 0.0 && a.top_p < 1.0;
    uint32_t c[4] = {(uint32_t)r, (uint32_t)((uint64_t)r >> 32), (uint32_t)a.offset,
                     (uint32_t)(a.offset >> 32)};
    philox4x32_10(c, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
    const double u01 = (double)(c[0] >> 8) * 5.9604644775390625e-8;  // 2^-24

    if (listed) {
      uint32_t tok_bits;
      list_draw<Tag>(cs, sh_s, cs.n, kth, need_k, use_p, a.top_p, iT, m,
                     float_key<KB>(load_one<Tag>(row, bi)), u01, tok, logq, tok_bits);
    } else {
      auto cand = [&](int e, uint32_t key) {
        return !use_k || key > kth || (key == kth && (need_k >= cnt_k || e <= cut_k));
      };

      // 3. Z over the candidates (the whole row's online sum without top-k).
      float zs = os;  // relative to the row maximum
      if (use_k) {
        zs = 0.0f;
        for_slabs<Tag>(row, V, al16, nslab, [&](int, int e0, const uint32_t (&u)[VEC], auto full) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            if ((full || e0 + i < V) && cand(e0 + i, float_key<KB>(u[i])))
              zs += expf(Bits<Tag>::val(u[i]) * iT - m);
          }
        });
        float v1[1] = {zs};
        block_sum<SNT, 1, float>(v1, sh_s);
        zs = v1[0];
      }
      const float inv_z = 1.0f / zs;
      auto ex = [&](uint32_t b) {
        float e = expf(Bits<Tag>::val(b) * iT - m);
        asm volatile("" : "+v"(e));
        return e;
      };
      auto prob = [&](uint32_t b) { return ex(b) * inv_z; };

      // 4. top-p: radix select over fixed-point mass in descending key order.
      bool p_found = false;
      uint32_t pth = 0;
      unsigned long long n_keep = 0, cnt_p = 0;
      int cut_p = -1;
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
          for_slabs<Tag>(row, V, al16, nslab, [&](int, int e0, const uint32_t (&u)[VEC], auto full) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
              const uint32_t key = float_key<KB>(u[i]);
              if ((full || e0 + i < V) && (key & pmask) == prefix && cand(e0 + i, key)) {
                const unsigned long long fx =
                    (unsigned long long)((double)prob(u[i]) * kMassScale);
                atomicAdd(&hist[(key >> shift) & 255u], 1u);
                atomicAdd(&histm[(key >> shift) & 255u], fx);
              }
            }
          });
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
          if (shift == 0) {
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
            cut_p = vocab_search<Tag, false>(
                row, V, al16, nslab,
                [&](int e, uint32_t b) {
                  const uint32_t key = float_key<KB>(b);
                  return (key == pth && cand(e, key)) ? 1.0f : 0.0f;
                },
                [&](double) { return nth; }, sh);
          }
        }
      }
      auto kept = [&](int e, uint32_t key) {
        return !p_found || key > pth ||
               (key == pth && (n_keep >= cnt_p || (n_keep > 0 && e <= cut_p)));
      };
      // q weight of a top-k candidate, floored; 0 outside the candidates
      auto qw = [&](int e, uint32_t b) {
        const uint32_t key = float_key<KB>(b);
        return cand(e, key) ? fmaxf(kept(e, key) ? ex(b) * inv_z : 0.0f, 1e-9f) : 0.0f;
      };

      // 5. inverse CDF with this row's uniform.
      __shared__ double sh_total;
      auto target = [&](double total) {
        if (tid == 0) sh_total = total;
        return u01 * total;
      };
      auto draw = [&](auto wfn, auto all_positive) {
        tok = vocab_search<Tag, decltype(all_positive)::value>(row, V, al16, nslab, wfn, target,
                                                               sh);
        const double qtot = sh_total;
        __syncthreads();
        if (tok < 0 || tok >= V) tok = bi;  // no positive weight: cannot happen, q >= 1e-9
        if (tid == 0) logq = (float)(log((double)wfn(tok, load_one<Tag>(row, tok))) - log(qtot));
      };
      if (!use_k && !p_found) {
        // The floored softmax max(p, 1e-9) as sample_resident_kernel's
        // mixture: p with probability 1 / (1 + G), else the floor's excess
        // g = max(1e-9 - p, 0), chosen by the component uniform u1; G takes
        // a pass of its own only when u1 < V * 1e-9 (>= G / (1 + G)) or
        // log q is asked for.
        const float lz = log2f(zs);
        auto rho_of = [&](uint32_t b) {
          return exp2_hw(__builtin_fmaf(Bits<Tag>::val(b) - bx, c2, -lz));
        };
        const double u1 = (double)(((uint64_t)c[1] << 21) | (c[2] >> 11)) * 0x1p-53;
        const bool near = u1 < (double)V * 1.001e-9;
        double G = 0.0;
        if (a.logq || near) {
          float gs = 0.0f;
          for_slabs<Tag>(row, V, al16, nslab, [&](int, int e0, const uint32_t (&u)[VEC], auto full) {
#pragma unroll
            for (int i = 0; i < VEC; ++i)
              if (full || e0 + i < V) gs += fmaxf(1e-9f - rho_of(u[i]), 0.0f);
          });
          double t[1] = {(double)gs};
          block_sum<SNT, 1, double>(t, sh.wave_tot);
          G = t[0];
        }
        const bool use_g = near && u1 < G / (1.0 + G);
        tok = vocab_search<Tag, false>(
            row, V, al16, nslab,
            [&](int, uint32_t b) {
              const float p = rho_of(b);
              return use_g ? fmaxf(1e-9f - p, 0.0f) : p;
            },
            target, sh);
        __syncthreads();
        if (tok < 0 || tok >= V) tok = bi;  // no positive weight: cannot happen with p
        if (tid == 0 && a.logq)
          logq = (float)(log((double)fmaxf(rho_of(load_one<Tag>(row, tok)), 1e-9f)) - log1p(G));
      } else {
        draw(qw, std::false_type{});
      }
    }
    // The token's S_other from pass 1: the sum without the maximum when the
    // token is the argmax, else Z minus the token's own term.  S_other then
    // holds the maximum's term 1 and e_tok <= 1, so the difference loses at
    // most one bit.
    if (tok != bi)
      s_other = os - exp2_hw((Bits<Tag>::val(load_one<Tag>(row, tok)) - bx) * c2);
  }

  // 6. log_softmax(x / T) at the token, as the training row kernels form it:
  // finish_row of the maximum, the sum over the other columns and the
  // token's own value.
  if (tid == 0) {
    const float xt = Bits<Tag>::val(load_one<Tag>(row, tok)) * iT;
    const RowLogprob<float> fr = finish_row<float>(m, s_other, xt);
    a.token[r] = tok;
    a.logp[r] = fr.logp;
    if (a.logq) a.logq[r] = logq;
  }
}

template <class Tag>
__global__ __launch_bounds__(SNT) void sample_kernel(SampleArgs a) {
  __shared__ CandShared cs;
  __shared__ uint32_t hist[256];
  const int64_t r = blockIdx.x;
  if (r >= a.B) return;
  // A fill-in launch redoes the rows the register-resident nucleus path
  // handed over (token slot -1); the others return at once.
  if (a.fill_in && __builtin_nontemporal_load(&a.token[r]) != -1) return;
  sample_row<Tag>(a, r, cs, hist);
}

template <class Tag>
int launch_sample(const SampleArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((sample_kernel<Tag>), dim3((unsigned)a.B), dim3(SNT), 0, st, a);
  return check_launch("sample_kernel");
}

// ---------------------------------------------------------------------------
// Register-resident rows of 16-bit logits made of whole 16-byte vectors
// (V % 8 == 0, rows 16-byte aligned, V <= 8 * 1024 * RES_MAX_SLABS).  Lane j
// holds vector k*1024 + j of its row in four VGPRs per slab k (the
// sample_kernel layout), so the row is read from memory once.  Greedy
// decoding and plain sampling run sample_blocks_kernel (below); top-k
// (top_k <= the lanes holding row data) with or without top-p runs
// sample_resident_kernel:
//   A. as the slab loads land: the lane's first maximum (value and slab) and
//      its online sum of exp((x - max) / T); one LDS exchange gives the row
//      maximum, Z and the lowest-index argmax;
//   K. the k-th largest lane maximum t0 (a radix select over the 1024 lane
//      maxima), every entry >= t0 gathered into the LDS list (past 1024
//      entries into a 3072-entry tail, then cut at the exact k-th key over
//      all of them); a list of at most 64 entries is drawn with the work
//      split for a short list (small_list_draw), a longer one is put in
//      vocabulary order (counting sort by 512-entry block), its exact k-th
//      key taken by a radix select, and list_draw applies the ties, top-p
//      and the draw; a row whose list still overflows takes the streaming
//      path (sample_row) in the same launch;
//   C. the sampled token's S_other: for the argmax, the sum over every other
//      entry relative to the row maximum, formed by the argmax lane's wave
//      (the other lanes' sweep-A sums, the argmax lane's entries shared out
//      over the wave through LDS); no subtraction, so the log-prob of a
//      dominant token keeps its relative precision.  Any other token: Z - e_tok.
constexpr int RES_MAX_SLABS = 20;  // V <= 163840

template <class Tag>
__device__ __forceinline__ void unpack8(const u32x4& u, float (&v)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = Bits<Tag>::val(w[i] & 0xffffu);
    v[2 * i + 1] = Bits<Tag>::val(w[i] >> 16);
  }
}

// IEEE maximum (v_maximum3_f32): NaN propagates, so the raw loaded values need
// no quieting first; a NaN row is flagged through its sum either way.
__device__ __forceinline__ float mx(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max8(const float (&v)[8]) {
  return mx(mx(mx(v[0], v[1]), mx(v[2], v[3])), mx(mx(v[4], v[5]), mx(v[6], v[7])));
}
// 4 x the slot of 16-bit entry HI (the dword's high half) or low of w among
// a top-p pass's per-key counts, in one multiply-add on the raw bits: POS,
// bits * 4 + c (every counted key a positive number's); otherwise
// (every counted key a negative number's) c - 4 * bits as a signed 16-bit
// value.
template <bool POS, bool HI>
__device__ __forceinline__ uint32_t slot4(uint32_t w, uint32_t c) {
  uint32_t r;
  if constexpr (POS) {
    if constexpr (HI) asm("v_mad_u32_u16 %0, %1, 4, %2 op_sel:[1,0,0,0]" : "=v"(r) : "v"(w), "v"(c));
    else asm("v_mad_u32_u16 %0, %1, 4, %2" : "=v"(r) : "v"(w), "v"(c));
  } else {
    if constexpr (HI) asm("v_mad_i32_i16 %0, %1, -4, %2 op_sel:[1,0,0,0]" : "=v"(r) : "v"(w), "v"(c));
    else asm("v_mad_i32_i16 %0, %1, -4, %2" : "=v"(r) : "v"(w), "v"(c));
  }
  return r;
}

__device__ __forceinline__ float sum8(const float (&e)[8]) {
  return ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
}

// The k-th largest of NK 16-bit keys per thread (keys whose valid flag is
// false take no part; 1 <= k <= the number of valid keys): MSB-first radix
// select, 8 bits per pass, over an LDS histogram of 256 bins.
template <int NK>
__device__ __forceinline__ uint32_t block_kth_keys16(const uint32_t (&key)[NK],
                                                     const bool (&valid)[NK], int k,
                                                     uint32_t* hist, uint32_t* sh_digit,
                                                     uint32_t* sh_above) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t prefix = 0, pmask = 0;
  uint32_t kk = (uint32_t)k;
  for (int shift = 8; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NK; ++j)
      if (valid[j] && (key[j] & pmask) == prefix) atomicAdd(&hist[(key[j] >> shift) & 255u], 1u);
    __syncthreads();
    if (wave == 0) {
      // lane l owns bins 4l..4l+3; the count above a bin is a suffix sum.
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
        if (above < kk && kk <= above + c[b]) {
          *sh_digit = 4 * lane + b;
          *sh_above = above;
        }
        above += c[b];
      }
    }
    __syncthreads();
    const uint32_t d = *sh_digit;
    kk -= *sh_above;
    prefix |= d << shift;
    pmask |= 255u << shift;
    __syncthreads();
  }
  return prefix;
}
__device__ __forceinline__ uint32_t block_kth_key16(uint32_t key, bool valid, int k,
                                                    uint32_t* hist, uint32_t* sh_digit,
                                                    uint32_t* sh_above) {
  const uint32_t ks[1] = {key};
  const bool vs[1] = {valid};
  return block_kth_keys16<1>(ks, vs, k, hist, sh_digit, sh_above);
}

// A value known to be the same in every active lane, moved to scalar
// registers (the compiler cannot prove values read back from LDS uniform,
// and the register-resident kernels have no vector registers to spare).
__device__ __forceinline__ float uni(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ double uni(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)b);
  const unsigned hi = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(b >> 32));
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// DPP row shift right by N lanes of a float64 (both halves moved alike); a
// lane whose source lies before its row's start reads 0.
template <int N>
__device__ __forceinline__ double row_shr_d(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const unsigned lo =
      (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)b, 0x110 + N, 0xF, 0xF, true);
  const unsigned hi =
      (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), 0x110 + N, 0xF, 0xF, true);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Inclusive prefix sums of v within each row of 16 lanes.
__device__ __forceinline__ double row_scan_d(double v) {
  v += row_shr_d<1>(v);
  v += row_shr_d<2>(v);
  v += row_shr_d<4>(v);
  v += row_shr_d<8>(v);
  return v;
}

// Inclusive and exclusive float64 prefix sums over the wave in lane order,
// and the total.  Each lane's exclusive value is the previous lane's
// inclusive one (the same operands, the same operation), so the ranges
// [excl, incl) of consecutive lanes tile [0, total).
__device__ __forceinline__ void wave_scan_d(double v, double& incl, double& excl, double& total) {
  const int lane = threadIdx.x & 63, row = lane >> 4;
  const double in = row_scan_d(v);
  const double pin = row_shr_d<1>(in);  // the previous lane's, 0 at a row start
  const double o1 = readlane_d(in, 15);
  const double o2 = o1 + readlane_d(in, 31);
  const double o3 = o2 + readlane_d(in, 47);
  const double off = row == 0 ? 0.0 : (row == 1 ? o1 : (row == 2 ? o2 : o3));
  incl = row == 0 ? in : off + in;
  excl = (lane & 15) == 0 ? off : (row == 0 ? pin : off + pin);
  total = o3 + readlane_d(in, 63);
}

// The lane whose range [base + excl, base + incl) of weight w > 0 holds
// target, else (rounding left target at or past the end) the last lane with
// w > 0, else -1; start = that lane's base + excl.
__device__ __forceinline__ int wave_claim(double w, double lo, double hi, double target,
                                          double& start) {
  const unsigned long long hit = __ballot(w > 0.0 && lo <= target && target < hi);
  const unsigned long long pos = __ballot(w > 0.0);
  const int l = hit ? __builtin_ctzll(hit) : (pos ? 63 - __builtin_clzll(pos) : -1);
  start = l >= 0 ? readlane_d(lo, l) : 0.0;
  return l;
}

// Pairwise sums of small_list_draw, entry i (lane i) against partners j of
// wave w's four (4w .. 4w + 3).
struct SmallShared {
  int cnt[SWAVES][64];      // rank by index | keys above << 8 | keys equal << 16
  uint32_t key[64];         // the candidates in index order: key,
  double mass[64];          // fixed-point probability (an integer < 2^53; -1: not a candidate)
  double above[SWAVES][64];  // top-p: mass of the candidates with a larger key,
  double at[SWAVES][64];     // with the same key,
  int eqc[SWAVES][64];       // how many with the same key | how many of them before i << 8
  int tok;
  float logq;
  uint32_t bits;
};

// list_draw for a list of n <= 64 entries (top-k up to a few dozen, as
// usual), with the exact k-th key (k = kq) found on the list first: every
// entry whose key is above the k-th key and the first need_k at it, lowest
// index first, are the candidates.  The rules are list_draw's; the work is
// laid out for a short list.  Entry i is lane i of every wave, and the
// pairwise counts (the rank by index, the keys above and equal, then top-p's
// masses above and at a key, as exact integers in float64) are split over
// the 16 waves, four partners each.  Wave 0 sums them, puts the entries in
// index order through LDS, forms Z and the candidates' probabilities over
// the wave and draws by a float64 scan over the wave: three workgroup
// barriers and no serial loop over the list.  Every thread returns the
// token, log q(token) and the token's stored bits.
template <class Tag>
__device__ __forceinline__ void small_list_draw(CandShared& cs, SmallShared& ss, int n, int kq,
                                                bool use_p, double top_p, float iT, float m,
                                                uint32_t max_key, double u01, int& tok,
                                                float& logq, uint32_t& tok_bits) {
  constexpr int KB = Bits<Tag>::KB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool have = lane < n;
  {
    const int e0 = have ? cs.idx[lane] : 0x7fffffff;
    const uint32_t k0 = float_key<KB>(have ? cs.bits[lane] : 0u);
    int rank = 0, gt = 0, eq = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = 4 * wave + q;  // wave-uniform
      if (j < n) {
        const int ej = __builtin_amdgcn_readlane(e0, j);
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)k0, j);
        rank += ej < e0 ? 1 : 0;
        gt += kj > k0 ? 1 : 0;
        eq += kj == k0 ? 1 : 0;
      }
    }
    ss.cnt[wave][lane] = rank | (gt << 8) | (eq << 16);
  }
  __syncthreads();
  // Wave 0: the k-th key, the entries in index order, the candidates and
  // their probabilities.
  float pc = 0.0f;
  bool cand = false;
  int se = 0;
  uint32_t sb = 0u, sk = 0u;
  if (wave == 0) {
    int rank = 0, gt = 0, eq = 0;
#pragma unroll
    for (int w = 0; w < SWAVES; ++w) {
      const int c = ss.cnt[w][lane];
      rank += c & 255;
      gt += (c >> 8) & 255;
      eq += c >> 16;
    }
    // The k-th key: an entry with fewer than k keys above it and at least
    // k at or above it (every such entry has the same key and counts).
    const uint32_t k0 = float_key<KB>(have ? cs.bits[lane] : 0u);
    const unsigned long long kh = __ballot(have && gt < kq && kq <= gt + eq);
    const int kl = kh ? __builtin_ctzll(kh) : 0;
    const uint32_t kth = (uint32_t)__builtin_amdgcn_readlane((int)k0, kl);
    const int need_k = kq - __builtin_amdgcn_readlane(gt, kl);
    if (have) {
      cs.sidx[rank] = cs.idx[lane];
      cs.sbits[rank] = cs.bits[lane];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    se = have ? cs.sidx[lane] : 0;
    sb = have ? cs.sbits[lane] : 0u;
    sk = float_key<KB>(sb);
    const bool tie = have && sk == kth;
    const int tie_rank = __popcll(__ballot(tie) & ((1ull << lane) - 1ull));
    cand = have && (sk > kth || (tie && tie_rank < need_k));
    // Z over the candidates, with the general path's exp(x/T - m).
    const float ev = cand ? expf(Bits<Tag>::val(sb) * iT - m) : 0.0f;
    pc = ev * (1.0f / wave_sum_dpp(ev));
    ss.key[lane] = sk;
    ss.mass[lane] = cand ? (double)(unsigned long long)((double)pc * kMassScale) : -1.0;
  }
  bool keep = true;
  if (use_p) {
    // The threshold group: the first key, in descending order, whose
    // inclusive fixed-point mass passes P (the row maximum is always kept);
    // ties in it are kept lowest index first.  Masses are integers below
    // 2^52 summing to at most about 2^52, exact in float64.
    __syncthreads();
    {
      const uint32_t ki = ss.key[lane];
      double ab = 0.0, at = 0.0;
      int c = 0, before = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = 4 * wave + q;  // wave-uniform
        const double mj = j < n ? ss.mass[j] : -1.0;
        if (mj >= 0.0) {  // a candidate (its mass may round to 0)
          const uint32_t kj = ss.key[j];
          ab += kj > ki ? mj : 0.0;
          const bool same = kj == ki;
          at += same ? mj : 0.0;
          c += same ? 1 : 0;
          before += (same && j < lane) ? 1 : 0;
        }
      }
      ss.above[wave][lane] = ab;
      ss.at[wave][lane] = at;
      ss.eqc[wave][lane] = c | (before << 8);
    }
    __syncthreads();
    if (wave == 0) {
      double A = 0.0, Ms = 0.0;
      int C = 0, tr = 0;
#pragma unroll
      for (int w = 0; w < SWAVES; ++w) {
        A += ss.above[w][lane];
        Ms += ss.at[w][lane];
        const int c = ss.eqc[w][lane];
        C += c & 255;
        tr += c >> 8;
      }
      const unsigned long long P = (unsigned long long)(top_p * kMassScale);
      const unsigned long long Ai = (unsigned long long)A, Mi = (unsigned long long)Ms;
      const unsigned long long fh = __ballot(cand && Mi > 0 && Ai <= P && P < Ai + Mi);
      if (fh) {
        const int fl = __builtin_ctzll(fh);
        const uint32_t pth = (uint32_t)__builtin_amdgcn_readlane((int)sk, fl);
        const unsigned long long A0 = (unsigned long long)readlane_d(A, fl);
        const unsigned long long M0 = (unsigned long long)readlane_d(Ms, fl);
        const unsigned long long C0 = (unsigned long long)__builtin_amdgcn_readlane(C, fl);
        const unsigned long long each = M0 / C0;  // equal keys, equal mass
        unsigned long long n_keep = each > 0 ? (P - A0) / each : C0;
        if (pth == max_key && n_keep == 0) n_keep = 1;
        keep = sk > pth ||
               (sk == pth && (n_keep >= C0 || (n_keep > 0 && (unsigned long long)tr < n_keep)));
      }
    }
  }
  if (wave == 0) {
    // Inverse CDF over the candidates in vocabulary order; the last
    // candidate takes a target that rounding leaves past the end.
    const float wf = cand ? fmaxf(keep ? pc : 0.0f, 1e-9f) : 0.0f;
    double incl, excl, tot;
    wave_scan_d((double)wf, incl, excl, tot);
    const double tgt = u01 * tot;
    double start;
    const int pl = wave_claim((double)wf, excl, incl, tgt, start);
    if (lane == pl) {
      ss.tok = se;
      ss.bits = sb;
      ss.logq = (float)(log((double)wf) - log(tot));
    }
  }
  __syncthreads();
  tok = ss.tok;
  logq = ss.logq;
  tok_bits = ss.bits;
}

template <class Tag, int SL>
__global__ __launch_bounds__(SNT) void sample_resident_kernel(SampleArgs a) {
  static_assert(Tag::VEC == 8, "16-bit rows");
  __shared__ CandShared cs;  // top-k's candidate list
  __shared__ uint32_t hist[256];
  __shared__ uint32_t sh_digit, sh_above;
  __shared__ int blk_base[SL * SWAVES];  // a longer list's block counts, then bases
  __shared__ float sh_z[SWAVES];
  __shared__ float sh_m[SWAVES], sh_s[SWAVES];
  __shared__ int sh_i[SWAVES];
  __shared__ u32x4 arg_row[SL];  // the argmax lane's registers (sweep C)
  // A short list's pairwise sums (small_list_draw), or an overflowing
  // gather's tail (rs.ovf): never both in one row.
  __shared__ union {
    SmallShared ss;
    struct {
      int idx[OVF];
      uint32_t bits[OVF];
    } ovf;
  } rs;
  SmallShared& ss = rs.ss;

  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int V = (int)a.V;
  const int nvec = V >> 3;
  const int nslab = (nvec + SNT - 1) / SNT;
  const int nfull = nvec / SNT;  // slabs whose every lane lies inside the row
  const float NEG = -__builtin_huge_valf();
  const typename Tag::S* row = static_cast<const typename Tag::S*>(a.logits) + (int64_t)r * a.stride;
  const __amdgpu_buffer_rsrc_t src = row_rsrc(row, (uint32_t)V * 2u);
  u32x4 x[SL];
#pragma unroll
  for (int k = 0; k < SL; ++k)
    x[k] = __builtin_amdgcn_raw_buffer_load_b128(src, tid * 16, k * SNT * 16, kAuxLoad);

  const float iT = 1.0f / a.temp;
  const float c2 = iT * kLog2e;  // exp(y / T) = 2^(y * c2)

  // A. The lane's first maximum, the slab it lies in, and the sum of
  // exp((x - max) / T) over the lane's entries, slab by slab as they land.
  // fmaxf skips NaN; NaN and +inf reach the sum and flag the row.
  float lm = NEG, ls = 0.0f;
  int lk = 0;
  // Each slab's lane maximum (a value of the row, so 16 bits hold it
  // exactly), two slabs per register: the top-k gather tests these first.
  uint32_t mk[(SL + 1) / 2] = {};
#pragma unroll
  for (int k = 0; k < SL; ++k) {
    if (k < nslab) {
      if (k >= nfull) {
        // The row's last, partial slab: lanes past the end read zeros and
        // hold -inf from here on (the empty asm keeps this a branch rather
        // than a select in every slab).
        asm volatile("");
        if (k * SNT + tid >= nvec) x[k] = u32x4{Bits<Tag>::NEG_INF, Bits<Tag>::NEG_INF,
                                                Bits<Tag>::NEG_INF, Bits<Tag>::NEG_INF};
      }
      float v[8];
      unpack8<Tag>(x[k], v);
      const float mc = max8(v);
      mk[k >> 1] |= (Bits<Tag>::bits_of(mc) & 0xffffu) << (16 * (k & 1));
      lk = mc > lm ? k : lk;
      const float mn = fmaxf(lm, mc);
      const float mg = fmaxf(mn, -__FLT_MAX__);
      float e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = exp2_hw((v[i] - mg) * c2);
      ls = __builtin_fmaf(ls, exp2_hw((lm - mg) * c2), sum8(e));
      lm = mn;
    }
  }
  // Per wave: maximum, sum relative to it, and the lowest index holding it
  // (found in the one slab where each such lane first met its maximum).
  const float wm = wave_max_dpp(lm);
  const float ws = wave_sum_dpp(ls * exp2_hw((lm - fmaxf(wm, -__FLT_MAX__)) * c2));
  int ci = 0x7fffffff;
  if (lm == wm && wm > NEG) {
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      if (k == lk) {
        float v[8];
        unpack8<Tag>(x[k], v);
        int ic = 7;
#pragma unroll
        for (int i = 6; i >= 0; --i) ic = v[i] == wm ? i : ic;
        ci = (k * SNT + tid) * 8 + ic;
      }
    }
  }
  const int wi = wave_min_dpp(ci);
  if (lane == 0) {
    sh_m[wave] = wm;
    sh_s[wave] = ws;
    sh_i[wave] = wi;
  }
  __syncthreads();
  float M = sh_m[0];
  for (int w = 1; w < SWAVES; ++w) M = fmaxf(M, sh_m[w]);
  const float Mg = fmaxf(M, -__FLT_MAX__);
  float Z = 0.0f;
  int bi = 0x7fffffff;
  for (int w = 0; w < SWAVES; ++w) {
    Z += sh_s[w] * exp2_hw((sh_m[w] - Mg) * c2);
    bi = sh_m[w] == M ? min(bi, sh_i[w]) : bi;
  }
  if (M == NEG || Z != Z || __builtin_fabsf(M * iT) == __builtin_huge_valf() || bi >= V) {
    if (tid == 0) {
      raise_flag(a.status, RRL_FLAG_BAD_PROBS);
      a.token[r] = bi < V ? bi : 0;
      a.logp[r] = __builtin_nanf("");
      if (a.logq) a.logq[r] = __builtin_nanf("");
    }
    return;
  }

  // The argmax lane's registers, for its wave's S_other (sweep C).
  if (tid == ((bi >> 3) & (SNT - 1))) {
#pragma unroll
    for (int k = 0; k < SL; ++k) arg_row[k] = x[k];  // -inf past the row's end
  }
  // Sweep C reads it in the same wave, after the top-k draw's barriers.
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  uint32_t c[4] = {(uint32_t)r, 0u, (uint32_t)a.offset, (uint32_t)(a.offset >> 32)};
  philox4x32_10(c, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
  const double u01 = (double)(c[0] >> 8) * 5.9604644775390625e-8;  // 2^-24

  int tok = bi;
  float logq = 0.0f;
  // K. Top-k (top_k <= the lanes holding row data, so every lane maximum
  // counts): the k-th largest lane maximum t0 has at least k entries at or
  // above it.  Those entries (a float compare: a superset of the keys >= t0
  // when -0 and +0 meet) go to the LDS list; the exact k-th key, its ties,
  // top-p and the draw are found on the list.  A row whose list overflows
  // takes the streaming path (sample_row) in the same launch.
  const int kq = (int)a.top_k;
  constexpr int KB = Bits<Tag>::KB;
  const uint32_t t0 = block_kth_key16(float_key<KB>(Bits<Tag>::bits_of(lm)), tid < nvec, kq,
                                      hist, &sh_digit, &sh_above);
  const uint32_t max_key = float_key<KB>(Bits<Tag>::bits_of(M));
  const float t0f = Bits<Tag>::val(key_bits<KB>(t0));
  // Every entry at or above t0, to the list in any order: the first KCAP in
  // cs, the next OVF in rs.ovf (free until a short list's draw).
  if (tid == 0) cs.n = 0;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < SL; ++k) {
    if (k < nslab) {
      // The slab's lane maximum decides whether any of its 8 entries is
      // listed (the row holds no NaN here: a NaN row left through its sum).
      const float mc = Bits<Tag>::val((mk[k >> 1] >> (16 * (k & 1))) & 0xffffu);
      const bool inside = k * SNT + tid < nvec;
      if (inside && mc >= t0f) {
        float v[8];
        unpack8<Tag>(x[k], v);
        const uint32_t w[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (v[i] >= t0f) {
            const int p = atomicAdd(&cs.n, 1);
            const int e = (k * SNT + tid) * 8 + i;
            const uint32_t b = (w[i >> 1] >> (16 * (i & 1))) & 0xffffu;
            if (p < KCAP) {
              cs.idx[p] = e;
              cs.bits[p] = b;
            } else if (p < KCAP + OVF) {
              rs.ovf.idx[p - KCAP] = e;
              rs.ovf.bits[p - KCAP] = b;
            }
          }
        }
      }
    }
  }
  __syncthreads();
  int n = cs.n;
  if (n > KCAP && n <= KCAP + OVF) {
    // The list overflows (top_k in the hundreds, where the k-th lane maximum
    // lies well below the k-th entry) but fits with its tail: the exact k-th
    // key over all n entries (up to four per thread), then the entries at
    // or above it back into cs.
    constexpr int NE = (KCAP + OVF + SNT - 1) / SNT;
    int ei[NE];
    uint32_t eb[NE], ek[NE];
    bool ev[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      const int q = tid + SNT * j;
      ev[j] = q < n;
      ei[j] = !ev[j] ? 0 : (q < KCAP ? cs.idx[q] : rs.ovf.idx[q - KCAP]);
      eb[j] = !ev[j] ? 0u : (q < KCAP ? cs.bits[q] : rs.ovf.bits[q - KCAP]);
      ek[j] = float_key<KB>(eb[j]);
    }
    const uint32_t kth = block_kth_keys16<NE>(ek, ev, kq, hist, &sh_digit, &sh_above);
    if (tid == 0) cs.n = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      if (ev[j] && ek[j] >= kth) {
        const int p = atomicAdd(&cs.n, 1);
        if (p < KCAP) {
          cs.idx[p] = ei[j];
          cs.bits[p] = eb[j];
        }
      }
    }
    __syncthreads();
    n = cs.n;  // past KCAP only through ties at the k-th key
  }
  if (n > KCAP) {
    // The list still overflows (coarse logits, many ties at the threshold):
    // this row takes the streaming path, re-reading it from memory, in this
    // launch.  (The registers' row is not needed past the gather.)
    sample_row<Tag>(a, r, cs, hist);
    return;
  }
  const bool use_p = a.top_p > 0.0 && a.top_p < 1.0;
  uint32_t tok_bits;
  if (n <= 64) {
    // A list of one wave's size (top-k up to a few dozen, as usual).
    small_list_draw<Tag>(cs, ss, n, kq, use_p, a.top_p, iT, M * iT, max_key, u01, tok, logq,
                         tok_bits);
  } else {
    // A longer list is put in vocabulary order by a counting sort on the
    // 512-entry block an index lies in (idx >> 9: bins in row order, a few
    // entries each), then a rank by index inside the bin.
    const int nb = (V + 511) >> 9;  // <= nslab * 16 entries of blk_base
    const bool have = tid < n;
    const int ei = have ? cs.idx[tid] : 0;
    const uint32_t eb = have ? cs.bits[tid] : 0u;
    for (int b = tid; b < nb; b += SNT) blk_base[b] = 0;
    __syncthreads();
    const int slot = have ? atomicAdd(&blk_base[ei >> 9], 1) : 0;
    __syncthreads();
    if (wave == 0) {
      constexpr int PER = (SL * SWAVES + 63) / 64;
      int c[PER], lsum = 0;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = lane * PER + j;
        c[j] = e < nb ? blk_base[e] : 0;
        lsum += c[j];
      }
      int incl = lsum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      int run = incl - lsum;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = lane * PER + j;
        if (e < nb) blk_base[e] = run;
        run += c[j];
      }
    }
    __syncthreads();
    int b0 = 0, b1 = 0;
    if (have) {
      const int bin = ei >> 9;
      b0 = blk_base[bin];
      b1 = bin + 1 < nb ? blk_base[bin + 1] : n;
      cs.sidx[b0 + slot] = ei;
    }
    __syncthreads();
    if (have) {
      int rank = b0;
      for (int j = b0; j < b1; ++j) rank += cs.sidx[j] < ei ? 1 : 0;
      cs.idx[rank] = ei;
      cs.bits[rank] = eb;
    }
    __syncthreads();
    // The exact k-th key of the list (which holds every entry at or above
    // it), and how many of its ties the top k keep.
    const uint32_t key = float_key<KB>(eb);
    const uint32_t kth = block_kth_key16(key, have, kq, hist, &sh_digit, &sh_above);
    int n_above = 0;
    (void)block_excl_count(have && key > kth, cs.wave_cnt, n_above);
    list_draw<Tag>(cs, sh_z, n, kth, kq - n_above, use_p, a.top_p, iT, M * iT, max_key, u01,
                   tok, logq, tok_bits, true);
  }
  const float xt_raw = Bits<Tag>::val(tok_bits);

  // C. S_other of the token and its log-prob, by the wave holding it.
  const int W = ((tok >> 3) & (SNT - 1)) >> 6;
  if (wave != W) return;
  float s_other;
  if (tok == bi) {
    // Every entry but the argmax itself, relative to the row maximum: the
    // other lanes of this wave add their sweep-A sums, and the argmax lane's
    // own entries are shared out over the wave through LDS (a few per lane).
    const int L = (tok >> 3) & (SNT - 1);
    float s = (tid == L || lm == NEG) ? 0.0f : (lm == M ? ls : ls * exp2_hw((lm - M) * c2));
    const uint16_t* er = reinterpret_cast<const uint16_t*>(arg_row);
#pragma unroll
    for (int m = 0; m < (8 * SL + 63) / 64; ++m) {
      const int t = lane + 64 * m;  // entry t & 7 of slab t >> 3
      if (t < 8 * nslab) {
        const float e = exp2_hw((Bits<Tag>::val(er[t]) - M) * c2);
        s += ((t >> 3) * SNT + L) * 8 + (t & 7) == tok ? 0.0f : e;
      }
    }
    float so = wave_sum_dpp(s);
    for (int w = 0; w < SWAVES; ++w)
      if (w != W) so += sh_s[w] * exp2_hw((sh_m[w] - M) * c2);
    s_other = so;
  } else {
    // Z holds the maximum's term 1 >= e_tok, so the difference loses at most a bit.
    s_other = Z - exp2_hw((xt_raw - M) * c2);
  }
  if (lane == 0) {
    const RowLogprob<float> fr = finish_row<float>(M * iT, s_other, xt_raw * iT);
    a.token[r] = tok;
    a.logp[r] = fr.logp;
    if (a.logq) a.logq[r] = logq;
  }
}


// ---------------------------------------------------------------------------
// Register-resident rows, greedy decoding and sampling without top-k / top-p
// (the reference's defaults), on block sums.  The row layout is
// sample_resident_kernel's (lane j holds vector k*1024 + j of slab k).  Block
// (k, w) is wave w's 512 entries of slab k; taken in (k, w) order the blocks
// are the row in vocabulary order.
//   A. as slab k lands, wave w adds 2^((x - R_w) c2) over its block into
//      S[k][w] (one hardware exponential per entry), against a reference R_w
//      fixed per wave: the maximum of its block of slab 0.  Each lane keeps
//      its first maximum, for the argmax.  Nothing per lane is kept for
//      later: a block is one number.
//   After the loads: M and the lowest-index argmax from the wave maxima;
//      block weights t[k][w] = S[k][w] 2^((R_w - M) c2), one per lane of 16
//      lanes per slab (a wave whose R_w lies more than 64 binary orders below
//      M first redoes its sums against M, so no block sum can have
//      overflowed) and the slab totals T_k as DPP row sums in float64; wave 0
//      alone then scans the T_k (Z is their total).
//   B. (sampling) the floored softmax max(p, 1e-9) as the mixture of p
//      (probability 1 / (1 + G)) and the floor's excess max(1e-9 - p, 0)
//      (probability G / (1 + G), G = sum of the excess), chosen by a second
//      uniform.  Wave 0 finds the slab holding target = u * total by a scan
//      of the slab totals and then the block by a scan of that slab's block
//      weights; the block's wave scans its lanes' sums (recomputed from
//      registers), and the claiming lane walks its own 8 entries.  Every
//      level tiles as wave_scan_d does, and the last positive slab, block,
//      lane or entry takes a target that rounding leaves past the end.  G
//      costs one exponential per entry, only when log q is asked for or the
//      component uniform is below V * 1e-9 >= G / (1 + G); the excess's block
//      sums are formed in the second case alone.
//   C. S_other of the token: for the argmax, Z less its own block's weight
//      (in float64) plus that block recomputed without it, so a dominant
//      token keeps its relative precision; any other token: Z - e_tok.
template <class Tag, int SL, bool TOPP>
__global__ __launch_bounds__(SNT) void sample_blocks_kernel(SampleArgs a) {
  static_assert(Tag::VEC == 8, "16-bit rows");
  static_assert(SL <= 64, "one lane per slab in wave 0's scan");
  __shared__ float blk_s[SL][SWAVES];   // S[k][w], later the excess's wave sums
  __shared__ float blk_r[SWAVES];       // R_w
  __shared__ double blk_t[SL][SWAVES];  // t[k][w]
  __shared__ double slab_tot[SL];       // T_k
  __shared__ double blk_g[SL][SWAVES];  // the excess's block sums (rare)
  __shared__ double slab_g[SL];
  __shared__ double red_ws[SWAVES];
  __shared__ float sh_m[SWAVES];
  __shared__ int sh_i[SWAVES];
  __shared__ double sh_z, sh_run, sh_tgt;
  __shared__ int sh_ks, sh_ws, sh_sel;
  __shared__ float sh_x;
  // Top-p: counts per key, later each key's weight, then two slots of
  // fixed weights and a spare slot per lane
  __shared__ uint32_t bins[TOPP ? TOPP_BINS + 2 + 64 : 1];

  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int V = (int)a.V;
  const int nvec = V >> 3;
  const int nslab = (nvec + SNT - 1) / SNT;
  const int nfull = nvec / SNT;  // slabs whose every lane lies inside the row
  const float NEG = -__builtin_huge_valf();
  const typename Tag::S* row = static_cast<const typename Tag::S*>(a.logits) + (int64_t)r * a.stride;
  const __amdgpu_buffer_rsrc_t src = row_rsrc(row, (uint32_t)V * 2u);
  u32x4 x[SL];
#pragma unroll
  for (int k = 0; k < SL; ++k)
    x[k] = __builtin_amdgcn_raw_buffer_load_b128(src, tid * 16, k * SNT * 16, kAuxLoad);
  if constexpr (TOPP) {
    // the counts start at zero (ordered before their use by sweep A's barrier)
    for (int i = tid; i < TOPP_BINS; i += SNT) bins[i] = 0u;
  }

  const float iT = 1.0f / a.temp;
  const float c2 = iT * kLog2e;  // exp(y / T) = 2^(y * c2)

  // A.  fmaxf skips NaN in the lane maxima and in R_w; NaN and +inf reach
  // the block sums and flag the row.
  float lm = NEG, R = 0.0f;
  int lk = 0;
#pragma unroll
  for (int k = 0; k < SL; ++k) {
    if (k < nslab) {
      if (k >= nfull) {
        // The row's last, partial slab: lanes past the end read zeros and
        // hold -inf from here on (exponential 0).
        asm volatile("");
        if (k * SNT + tid >= nvec) x[k] = u32x4{Bits<Tag>::NEG_INF, Bits<Tag>::NEG_INF,
                                                Bits<Tag>::NEG_INF, Bits<Tag>::NEG_INF};
      }
      float v[8];
      unpack8<Tag>(x[k], v);
      const float mc = max8(v);
      lk = mc > lm ? k : lk;
      lm = fmaxf(lm, mc);
      if (k == 0) R = uni(fmaxf(wave_max_dpp(mc), -__FLT_MAX__));
      float e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = exp2_hw((v[i] - R) * c2);
      const float s = wave_sum_dpp(sum8(e));
      if (lane == 0) blk_s[k][wave] = s;
    }
  }
  // Per wave: the maximum and the lowest index holding it (found in the one
  // slab where each such lane first met its maximum).
  const float wm = wave_max_dpp(lm);
  int ci = 0x7fffffff;
  if (lm == wm && wm > NEG) {
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      if (k == lk) {
        float v[8];
        unpack8<Tag>(x[k], v);
        int ic = 7;
#pragma unroll
        for (int i = 6; i >= 0; --i) ic = v[i] == wm ? i : ic;
        ci = (k * SNT + tid) * 8 + ic;
      }
    }
  }
  const int wi = wave_min_dpp(ci);
  if (lane == 0) {
    sh_m[wave] = wm;
    sh_i[wave] = wi;
    blk_r[wave] = R;
  }
  if (tid == 0) sh_sel = -1;
  __syncthreads();
  // Lane l of every wave reads wave (l & 15)'s values.
  const float Rl = blk_r[lane & 15];
  const float mw = sh_m[lane & 15];
  const float M = uni(wave_max_dpp(mw));
  const int bi = uni(wave_min_dpp(mw == M ? sh_i[lane & 15] : 0x7fffffff));

  // A wave whose reference lies more than 64 binary orders below M (a later
  // slab rose far above its first) redoes its block sums against M; every
  // wave takes the same decision from the same LDS values.
  auto far_below = [&](float Rw) { return (M - Rw) * c2 > 64.0f; };
  if (__ballot(far_below(Rl)) != 0ull) {
    if (far_below(R)) {
#pragma unroll
      for (int k = 0; k < SL; ++k) {
        if (k < nslab) {
          float v[8];
          unpack8<Tag>(x[k], v);
          float e[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) e[i] = exp2_hw((v[i] - M) * c2);
          const float s = wave_sum_dpp(sum8(e));
          if (lane == 0) blk_s[k][wave] = s;
        }
      }
    }
    __syncthreads();
  }
  // Block weights, one per thread of the first nslab * 16, and the slab
  // totals as row sums (row k of 16 lanes is slab k).
  if (tid < nslab * SWAVES) {
    const int k = tid >> 4;
    const float t = blk_s[k][lane & 15] * exp2_hw(((far_below(Rl) ? M : Rl) - M) * c2);
    blk_t[k][lane & 15] = (double)t;
    const double T = row_scan_d((double)t);
    if ((lane & 15) == 15) slab_tot[k] = T;
  }
  __syncthreads();

  // The row's uniforms (sampling only): u01 places the draw, u1 picks the
  // mixture's component.
  double u01 = 0.0, u1 = 1.0;
  if (!a.greedy) {
    uint32_t c[4] = {(uint32_t)r, 0u, (uint32_t)a.offset, (uint32_t)(a.offset >> 32)};
    philox4x32_10(c, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
    u01 = uni((double)(c[0] >> 8) * 5.9604644775390625e-8);  // 2^-24
    u1 = uni((double)(((uint64_t)c[1] << 21) | (c[2] >> 11)) * 0x1p-53);
  }

  // Wave 0: Z, and for sampling the slab and block holding u01 * total of
  // the weights st (slab totals) and bt (block weights of slab k, lane w),
  // into sh_ks, sh_ws, sh_run (the total before the block) and sh_tgt.
  auto locate = [&](const double* st, auto bt) {
    const double ts = lane < nslab ? st[lane] : 0.0;
    double incl, excl, total;
    wave_scan_d(ts, incl, excl, total);
    const double target = u01 * total;
    double run;
    const int ks = wave_claim(ts, excl, incl, target, run);
    const double tb = ks >= 0 && lane < SWAVES ? bt(ks, lane) : 0.0;
    double bincl, bexcl, btot;
    wave_scan_d(tb, bincl, bexcl, btot);
    double brun;
    const int ws = wave_claim(tb, run + bexcl, run + bincl, target, brun);
    if (lane == 0) {
      sh_ks = ks;
      sh_ws = ks >= 0 ? ws : -1;
      sh_run = brun;
      sh_tgt = target;
    }
    return total;
  };
  if (wave == 0) {
    const double Z = a.greedy ? 0.0 : locate(slab_tot, [&](int k, int w) { return blk_t[k][w]; });
    if (lane == 0) {
      if (a.greedy) {
        double s = 0.0;
        for (int k = 0; k < nslab; ++k) s += slab_tot[k];
        sh_z = s;
      } else {
        sh_z = Z;
      }
    }
  }
  __syncthreads();
  const double Zd = uni(sh_z);

  if (M == NEG || Zd != Zd || __builtin_fabsf(M * iT) == __builtin_huge_valf() || bi >= V) {
    int tok_bad = bi < V ? bi : 0;
    if (a.greedy && Zd != Zd) {
      // Greedy decoding is torch.argmax, which ranks NaN above every number:
      // the row's first NaN is its token (entries past the row hold -inf).
      int fn = 0x7fffffff;
#pragma unroll
      for (int k = SL - 1; k >= 0; --k) {
        if (k < nslab) {
          float v[8];
          unpack8<Tag>(x[k], v);
#pragma unroll
          for (int i = 7; i >= 0; --i)
            if (v[i] != v[i]) fn = (k * SNT + tid) * 8 + i;
        }
      }
      fn = block_min_i32(fn);
      if (fn < V) tok_bad = fn;
    }
    if (tid == 0) {
      raise_flag(a.status, RRL_FLAG_BAD_PROBS);
      a.token[r] = tok_bad;
      a.logp[r] = __builtin_nanf("");
      if (a.logq) a.logq[r] = __builtin_nanf("");
    }
    return;
  }

  int tok = bi;
  float logq = 0.0f;
  bool q_from_p = false;  // log q from the token's log-prob and G
  float q_g = 0.0f;
  float xt_raw = M;  // the token's logit
  if (!a.greedy) {
    if constexpr (TOPP) {
      // P. Top-p without top-k (bfloat16 rows; every entry a candidate, so
      // those outside the nucleus keep the floor 1e-9).  The cut lies at or
      // above x_lo, where the mass of all V entries below it would be under
      // (1 - top_p) / 2.  One count per key from x_lo's up (LDS atomics, no
      // exponentials); the keys' fixed-point masses count * floor(p 2^52),
      // scanned in descending key order, give the threshold group as the
      // streaming kernel's radix select does; its ties are kept lowest index
      // first (the n_keep-th found from block counts in vocabulary order).
      // The counts then become each key's floored weight, and the block sums
      // of the weights (one LDS read per entry) place the draw as for plain
      // sampling.  A row whose keys from x_lo up outnumber the counts is left
      // to the fill-in launch.
      constexpr int KB = Bits<Tag>::KB;
      constexpr int NB = TOPP_BINS;
      constexpr int PB = NB / SNT;  // descending key positions per thread
      __shared__ unsigned long long red_u[SWAVES];
      __shared__ double blk_w[SL][SWAVES];
      __shared__ double slab_w[SL];
      __shared__ int cnt_b[SL * SWAVES];
      __shared__ int sh_found, sh_cut, sh_blk, sh_off;
      __shared__ uint32_t sh_pth;
      __shared__ unsigned long long sh_a0, sh_c0, sh_each;
      __shared__ double sh_tot;
      __shared__ float sh_lq;
      const float lz = uni(log2f((float)Zd));
      auto pn = [&](float v) { return exp2_hw(__builtin_fmaf(v - M, c2, -lz)); };  // p
      const uint32_t kmax = float_key<KB>(Bits<Tag>::bits_of(M));
      const float xlo =
          uni(M + (float)(log2((1.0 - a.top_p) * Zd / (2.0 * (double)V)) / (double)c2));
      // a key at or below x_lo's (the conversion truncates by less than one step)
      uint32_t klo = xlo > -__FLT_MAX__ ? float_key<KB>(Bits<Tag>::bits_of(xlo)) : 0u;
      klo = klo > 0u ? klo - 1u : 0u;
      // An entry's slot among the counts is its key - klo, counted when below
      // R = kmax - klo + 1.  When every key from klo to kmax is a positive
      // number's, or every one a negative number's, slot4 forms 4 x the slot
      // from the raw bits in one multiply-add.
      const bool pos = klo > 0x8000u, neg = kmax < 0x8000u;
      if (klo == 0u || kmax < klo || kmax - klo >= (uint32_t)NB || !(pos || neg)) {
        // The keys from x_lo up outnumber the counts (a flat row over many
        // binades) or cross zero: the fill-in launch that follows takes this
        // row.
        if (tid == 0) a.token[r] = -1;
        return;
      }
      const uint32_t R = kmax - klo + 1u;
      // 4 x the slot, from slot4's constant: POS 4 (0x8000 - klo), else
      // 4 (-1 - klo); a lane past the row's end (the last slab) takes one
      // that puts it far above 4 (R + 1).
      const uint32_t c_in = pos ? 4u * (0x8000u - klo) : 4u * (0xffffffffu - klo);
      const uint32_t c_out = pos ? 0xfff00000u : 0x80000000u;
      if (tid == 0) {
        sh_found = 0;
        sh_cut = 0x7fffffff;
      }
      // body(slab k's vector, k, the lane inside the row, its slot4 constant)
      // for every slab.  pick takes its operands by value: a conditional on
      // the two named constants would select between their addresses and
      // keep them, and the lambdas' captures, in scratch memory.
      auto pick = [](bool p, uint32_t u, uint32_t v) { return p ? u : v; };
      auto each_slab = [&](auto body) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < SL; ++k) {
          if (k < nslab) {
            const bool in_row = k < nfull || k * SNT + tid < nvec;
            body(x[k], k, in_row, pick(in_row, c_in, c_out));
          }
        }
      };
      // 4 x the slots of a vector's 8 entries (ps: the positive form)
      auto slots8 = [](u32x4 xv, uint32_t c, uint32_t (&t)[8], auto ps) __attribute__((always_inline)) {
        constexpr bool P_ = decltype(ps)::value;
        const uint32_t w[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          t[2 * j] = slot4<P_, false>(w[j], c);
          t[2 * j + 1] = slot4<P_, true>(w[j], c);
        }
      };
      // Counts per key from klo up (the counts were cleared at the start).
      const uint32_t R4 = 4u * R;
      const uint32_t spare = 4u * (uint32_t)(TOPP_BINS + 2 + lane);
      auto count = [&](auto ps) __attribute__((always_inline)) {
        each_slab([&](u32x4 xv, int, bool, uint32_t c) __attribute__((always_inline)) {
          uint32_t t[8];
          slots8(xv, c, t, ps);
          // Every lane adds: an entry outside the counts into the lane's own
          // spare slot past them (no branch per entry, no shared address).
#pragma unroll
          for (int i = 0; i < 8; ++i)
            atomicAdd(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(bins) +
                                                  (t[i] < R4 ? t[i] : spare)),
                      1u);
        });
      };
      if (pos) count(std::true_type{});
      else count(std::false_type{});
      __syncthreads();
      // Thread t holds descending positions 4t..4t+3 (key kmax - position).
      const unsigned long long P = (unsigned long long)(a.top_p * kMassScale);
      auto pkey = [&](int d) {  // p of the key at position d
        return pn(Bits<Tag>::val(key_bits<KB>(kmax - (uint32_t)d)));
      };
      // its fixed-point mass floor(p 2^52)
      auto fixed = [](float p) { return (unsigned long long)((double)p * kMassScale); };
      uint32_t c4[PB];
      unsigned long long lsum = 0;
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        const int d = tid * PB + j;
        c4[j] = d < (int)R ? bins[R - 1 - d] : 0u;
        lsum += c4[j] ? c4[j] * fixed(pkey(d)) : 0ull;
      }
      unsigned long long inc = lsum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long y = __shfl_up(inc, o, 64);
        if (lane >= o) inc += y;
      }
      if (lane == 63) red_u[wave] = inc;
      __syncthreads();
      // The masses above each position give the threshold group (the one
      // holding P) and, in place of the counts (every count has been read),
      // each key's floored weight: p if kept, else 1e-9; the group's p if
      // any of it is kept.  Slot R, where every entry below klo reads, holds
      // 1e-9 and slot R + 1 zero.  Block sums of the weights then need one
      // LDS read per entry instead of an exponential.
      unsigned long long above = inc - lsum;
      for (int w = 0; w < wave; ++w) above += red_u[w];
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        const int d = tid * PB + j;
        const float pj = pkey(d);
        const unsigned long long f = c4[j] ? fixed(pj) : 0ull, m = c4[j] * f;
        float wk = 1e-9f;
        if (above <= P && P - above >= m) {
          wk = fmaxf(pj, 1e-9f);  // every entry at this key kept
        } else if (c4[j] > 0 && above <= P) {  // one bin: the group holding P
          unsigned long long nk = f > 0 ? (P - above) / f : c4[j];
          if (d == 0 && nk == 0) nk = 1;  // the row maximum is always kept
          wk = nk > 0 ? fmaxf(pj, 1e-9f) : 1e-9f;
          sh_found = 1;
          sh_pth = kmax - (uint32_t)d;
          sh_a0 = above;
          sh_c0 = c4[j];
          sh_each = f;
        }
        if (d < (int)R) bins[R - 1 - d] = __float_as_uint(wk);
        above += m;
      }
      if (tid == 0) {
        bins[R] = __float_as_uint(1e-9f);
        bins[R + 1] = 0u;
      }
      __syncthreads();
      const bool found = sh_found != 0;
      const uint32_t pth = sh_pth;
      const float fth = Bits<Tag>::val(key_bits<KB>(pth));
      const unsigned long long C0 = sh_c0, each = sh_each;
      unsigned long long n_keep = found ? (each > 0 ? (P - sh_a0) / each : C0) : 0;
      // The first token in descending order (the row maximum) is always kept.
      if (found && pth == kmax && n_keep == 0) n_keep = 1;
      // Some but not all of the threshold group kept: lowest index first.
      const bool partial = found && n_keep > 0 && n_keep < C0;
      // The floored weight of each key tied at the threshold, and of a kept one.
      const float wth = n_keep > 0 ? fmaxf(pn(fth), 1e-9f) : 1e-9f;
      if (found) {
        // Block sums with every tie at wth (a lane past the row's end reads
        // slot R + 1, zero), and each block's count of ties.
        // Lane k keeps slab k's block sum and tie count until the end.
        const uint32_t tt4 = 4u * (pth - klo);
        float my_w = 0.0f;
        int my_c = 0;
        auto weigh = [&](auto ps) __attribute__((always_inline)) {
          each_slab([&](u32x4 xv, int k, bool in_row, uint32_t c) __attribute__((always_inline)) {
            const uint32_t Rk4 = in_row ? R4 : R4 + 4u;
            uint32_t t[8];
            slots8(xv, c, t, ps);
            float w8[8];
            int tot = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const uint32_t off = t[i] < Rk4 ? t[i] : Rk4;
              w8[i] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(bins) + off);
              tot += __popcll(__ballot(t[i] == tt4));
            }
            const float sw = wave_sum_dpp(sum8(w8));
            my_w = lane == k ? sw : my_w;
            my_c = lane == k ? tot : my_c;
          });
        };
        if (pos) weigh(std::true_type{});
        else weigh(std::false_type{});
        if (lane < nslab) {
          blk_w[lane][wave] = (double)my_w;
          cnt_b[lane * SWAVES + wave] = my_c;
        }
        __syncthreads();
        if (partial) {
          // Wave 0: the ties before each block in vocabulary order; a block's
          // ties past the n_keep-th drop from wth to 1e-9, and the block
          // holding the n_keep-th is recorded.
          if (wave == 0) {
            constexpr int PER = (SL * SWAVES + 63) / 64;
            const int E = nslab * SWAVES;
            const long long tk = (long long)n_keep - 1;
            const double drop = (double)wth - (double)1e-9f;
            int c[PER], ls_ = 0;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
              const int e = lane * PER + j;
              c[j] = e < E ? cnt_b[e] : 0;
              ls_ += c[j];
            }
            int incl = ls_;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
              const int y = __shfl_up(incl, o, 64);
              if (lane >= o) incl += y;
            }
            int run = incl - ls_;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
              const int e = lane * PER + j;
              if (c[j] > 0) {
                if (run <= tk && tk < run + c[j]) {
                  sh_blk = e;
                  sh_off = (int)(tk - run);
                }
                const long long kept =
                    (long long)n_keep - run < 0 ? 0 : std::min<long long>((long long)n_keep - run, c[j]);
                if (kept < c[j]) blk_w[e / SWAVES][e % SWAVES] -= (double)(c[j] - kept) * drop;
              }
              run += c[j];
            }
          }
          __syncthreads();
          // The n_keep-th tie itself: the recorded block's wave.
          const int kb2 = sh_blk / SWAVES, wb2 = sh_blk % SWAVES, off = sh_off;
          if (wave == wb2) {
            u32x4 xv = x[0];
#pragma unroll
            for (int k = 1; k < SL; ++k) xv = k == kb2 ? x[k] : xv;
            float v[8];
            unpack8<Tag>(xv, v);
            const bool inside = kb2 * SNT + tid < nvec;
            uint32_t below = 0;
            int h = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const unsigned long long m = __ballot(inside && v[i] == fth);
              below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo((uint32_t)m, below));
              h += (int)((m >> lane) & 1ull);
            }
            if ((int)below <= off && off < (int)below + h) {
              int seen = (int)below;
#pragma unroll
              for (int i = 0; i < 8; ++i) {
                if (inside && v[i] == fth) {
                  if (seen == off) sh_cut = (kb2 * SNT + tid) * 8 + i;
                  ++seen;
                }
              }
            }
          }
        }
      } else {
        // No threshold group (the fixed-point masses fall short of top_p):
        // every entry is kept.
#pragma unroll
        for (int k = 0; k < SL; ++k) {
          if (k < nslab) {
            const bool inside = k * SNT + tid < nvec;
            float v[8];
            unpack8<Tag>(x[k], v);
            float w8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) w8[i] = inside ? fmaxf(pn(v[i]), 1e-9f) : 0.0f;
            const float sw = wave_sum_dpp(sum8(w8));
            if (lane == 0) blk_w[k][wave] = (double)sw;
          }
        }
        __syncthreads();
      }
      // floored weight of entry e (logit v): p if kept, else 1e-9
      auto wq = [&](int e, float v) {
        const bool kept =
            !found || v > fth || (v == fth && (n_keep >= C0 || (n_keep > 0 && e <= sh_cut)));
        return kept ? fmaxf(pn(v), 1e-9f) : 1e-9f;
      };
      if (tid < nslab * SWAVES) {
        const int k = tid >> 4;
        const double T = row_scan_d(blk_w[k][lane & 15]);
        if ((lane & 15) == 15) slab_w[k] = T;
      }
      __syncthreads();
      if (wave == 0) {
        const double tot = locate(slab_w, [&](int k, int w) { return blk_w[k][w]; });
        if (lane == 0) sh_tot = tot;
      }
      __syncthreads();
      const int ks = uni(sh_ks), wsel = uni(sh_ws);
      if (wave == wsel) {
        const double run = uni(sh_run), target = uni(sh_tgt);
        u32x4 xv = x[0];
#pragma unroll
        for (int k = 1; k < SL; ++k) xv = k == ks ? x[k] : xv;
        float v[8];
        unpack8<Tag>(xv, v);
        const bool inside = ks * SNT + tid < nvec;
        float w8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w8[i] = inside ? wq((ks * SNT + tid) * 8 + i, v[i]) : 0.0f;
        const double lw = (double)sum8(w8);
        double incl, excl, total;
        wave_scan_d(lw, incl, excl, total);
        double lstart;
        const int lc = wave_claim(lw, run + excl, run + incl, target, lstart);
        if (lane == lc) {
          double cum = lstart;
          int pick = -1, lastp = 7;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            if (w8[i] > 0.0f) {
              lastp = i;
              if (pick < 0 && cum + (double)w8[i] > target) pick = i;
            }
            cum += (double)w8[i];
          }
          pick = pick >= 0 ? pick : lastp;
          float xp = v[0], wp = w8[0];
#pragma unroll
          for (int i = 1; i < 8; ++i) {
            xp = i == pick ? v[i] : xp;
            wp = i == pick ? w8[i] : wp;
          }
          sh_sel = (ks * SNT + tid) * 8 + pick;
          sh_x = xp;
          sh_lq = logf((float)((double)wp / sh_tot));
        }
      }
      __syncthreads();
      const int sel = sh_sel;
      if (sel >= 0) {  // else (not reached: every total is positive) the argmax
        tok = sel;
        xt_raw = sh_x;
        logq = sh_lq;
      }
    } else {
    const float lz = uni(log2f((float)Zd));
    const float K = uni(__builtin_fmaf(M, c2, lz));
    auto rho = [&](float v) { return exp2_hw((v - M) * c2); };  // Z p
    // The floor's side: p = 2^(x c2 - K) in one fma (its rounding only moves
    // the excess, a sum of at most V * 1e-9, by parts in 1e6).
    auto pf = [&](float v) { return exp2_hw(__builtin_fmaf(v, c2, -K)); };
    auto g_of = [&](float v) { return fmaxf(1e-9f - pf(v), 0.0f); };
    // min(p 1e9, 1) in one exponential: the clamp to [0, 1] is exp2's
    // output modifier (1e9 = 2^29.897352853986263)
    const float Kc = uni(K - 29.897352853986263f);
    auto pc = [&](float v) {
      return __builtin_amdgcn_fmed3f(exp2_hw(__builtin_fmaf(v, c2, -Kc)), 0.0f, 1.0f);
    };
    const bool want_q = a.logq != nullptr;
    const bool near = u1 < (double)V * 1.001e-9;
    // The excess's total G over this thread's entries, in units of 1e-9
    // (with the block sums of the near case).
    auto g_part = [&]() __attribute__((always_inline)) {
      float gs = 0.0f;
#pragma unroll
      for (int k = 0; k < SL; ++k) {
        if (k < nslab) {
          float v[8];
          unpack8<Tag>(x[k], v);
          // sum of max(1e-9 - p, 0) = 1e-9 (8 - sum of min(p 1e9, 1))
          float m[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) m[i] = pc(v[i]);
          float f = 8.0f - sum8(m);
          if (k >= nfull) {
            asm volatile("");
            if (k * SNT + tid >= nvec) f = 0.0f;  // -inf past the row's end is not floored
          }
          gs += f;
          if (near) {
            const float s = wave_sum_dpp(f);
            if (lane == 0) blk_s[k][wave] = s * 1e-9f;
          }
        }
      }
      return gs;
    };
    // The block's wave: its lanes' sums of the entry weights (0 past the
    // row's end), a float64 scan from the block's start, and the claiming
    // lane's own 8 entries, into sh_sel and sh_x.
    auto draw_in_block = [&](bool use_g) __attribute__((always_inline)) {
      const int ks = uni(sh_ks);
      const double run = uni(sh_run), target = uni(sh_tgt);
      // slab ks's vector, as masked ors (a chain of selects here would be
      // folded into a dynamic index into the registers, i.e. scratch)
      u32x4 xv = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int k = 0; k < SL; ++k) {
        const uint32_t m = k == ks ? 0xffffffffu : 0u;
        xv.x |= x[k].x & m;
        xv.y |= x[k].y & m;
        xv.z |= x[k].z & m;
        xv.w |= x[k].w & m;
      }
      float v[8];
      unpack8<Tag>(xv, v);
      const bool inside = ks * SNT + tid < nvec;
      float w8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w8[i] = !inside ? 0.0f : (use_g ? g_of(v[i]) : rho(v[i]));
      const double lw = (double)sum8(w8);
      double incl, excl, total;
      wave_scan_d(lw, incl, excl, total);
      double lstart;
      const int lc = wave_claim(lw, run + excl, run + incl, target, lstart);
      if (lane == lc) {
        double cum = lstart;
        int pick = -1, lastp = 7;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (w8[i] > 0.0f) {
            lastp = i;
            if (pick < 0 && cum + (double)w8[i] > target) pick = i;
          }
          cum += (double)w8[i];
        }
        pick = pick >= 0 ? pick : lastp;
        float xp = v[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) xp = i == pick ? v[i] : xp;
        sh_sel = (ks * SNT + tid) * 8 + pick;
        sh_x = xp;
      }
    };
    double G = 0.0;
    bool use_g = false;
    if (near) {
      // The draw may fall on the excess: G and its block sums first.
      double t[1] = {(double)g_part()};
      block_sum<SNT, 1, double>(t, red_ws);
      G = uni(t[0]) * 1e-9;
      use_g = u1 < G / (1.0 + G);
      if (use_g) {
        // The excess's block sums (written in the G pass) and slab totals,
        // then the same search over them.
        if (tid < nslab * SWAVES) {
          const int k = tid >> 4;
          const double tk = (double)blk_s[k][lane & 15];
          blk_g[k][lane & 15] = tk;
          const double T = row_scan_d(tk);
          if ((lane & 15) == 15) slab_g[k] = T;
        }
        __syncthreads();
        if (wave == 0) locate(slab_g, [&](int k, int w) { return blk_g[k][w]; });
        __syncthreads();
      }
    }
    if (wave == uni(sh_ws)) draw_in_block(use_g);
    if (!near && want_q) {
      // The draw needed p only, so the other waves summed the excess
      // meanwhile; G's barrier also publishes the draw.
      double t[1] = {(double)g_part()};
      block_sum<SNT, 1, double>(t, red_ws);
      G = uni(t[0]) * 1e-9;
    } else {
      __syncthreads();
    }
    const int sel = sh_sel;
    if (sel >= 0) {  // else (not reached: every total is positive) the argmax
      tok = sel;
      xt_raw = sh_x;
    }
    // log q(token) = log(max(p_tok, 1e-9)) - log(1 + G), from the token's
    // log-prob at the end.
    q_from_p = want_q;
    q_g = (float)G;
    }
  }

  // C. S_other of the token and its log-prob.
  const int tb = (bi >> 3) & (SNT - 1);  // the argmax's lane
  const int kb = (bi >> 3) / SNT;        // and slab
  const int W = tok == bi ? tb >> 6 : 0;
  if (wave != W) return;
  float s_other;
  if (tok == bi) {
    u32x4 xv = x[0];
#pragma unroll
    for (int k = 1; k < SL; ++k) xv = k == kb ? x[k] : xv;
    float v[8];
    unpack8<Tag>(xv, v);
    float e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = (tid == tb && i == (bi & 7)) ? 0.0f : exp2_hw((v[i] - M) * c2);
    const float sb = wave_sum_dpp(sum8(e));
    s_other = (float)((Zd - blk_t[kb][W]) + (double)sb);
  } else {
    s_other = (float)(Zd - (double)exp2_hw((xt_raw - M) * c2));
  }
  if (lane == 0) {
    const RowLogprob<float> fr = finish_row<float>(M * iT, s_other, xt_raw * iT);
    a.token[r] = tok;
    a.logp[r] = fr.logp;
    // log(max(p, 1e-9)) = max(log p, log 1e-9)
    if (q_from_p) logq = fmaxf(fr.logp, -20.723265836946411f) - log1pf(q_g);
    if (a.logq) a.logq[r] = logq;
  }
}

template <class Tag, int SL>
int launch_resident_sl(const SampleArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((sample_resident_kernel<Tag, SL>), dim3((unsigned)a.B), dim3(SNT), 0, st, a);
  return check_launch("sample_resident_kernel");
}

template <class Tag>
int launch_sample_resident(const SampleArgs& a, int nslab, hipStream_t st) {
  if (nslab <= 4) return launch_resident_sl<Tag, 4>(a, st);
  if (nslab <= 8) return launch_resident_sl<Tag, 8>(a, st);
  if (nslab <= 12) return launch_resident_sl<Tag, 12>(a, st);
  if (nslab <= 16) return launch_resident_sl<Tag, 16>(a, st);
  return launch_resident_sl<Tag, RES_MAX_SLABS>(a, st);
}

template <class Tag, int SL, bool TOPP>
int launch_blocks_sl(const SampleArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((sample_blocks_kernel<Tag, SL, TOPP>), dim3((unsigned)a.B), dim3(SNT), 0, st,
                     a);
  return check_launch("sample_blocks_kernel");
}

template <class Tag, bool TOPP>
int launch_sample_blocks(const SampleArgs& a, int nslab, hipStream_t st) {
  if (nslab <= 4) return launch_blocks_sl<Tag, 4, TOPP>(a, st);
  if (nslab <= 8) return launch_blocks_sl<Tag, 8, TOPP>(a, st);
  if (nslab <= 12) return launch_blocks_sl<Tag, 12, TOPP>(a, st);
  if (nslab <= 16) return launch_blocks_sl<Tag, 16, TOPP>(a, st);
  return launch_blocks_sl<Tag, RES_MAX_SLABS, TOPP>(a, st);
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
  // Plain sampling and greedy decoding of whole-vector, 16-byte aligned
  // 16-bit rows hold the row in registers; everything else streams it.
  const bool use_k = top_k > 0 && top_k < V;
  const bool use_p = top_p > 0.0 && top_p < 1.0;
  const int64_t nvec = V / 8;
  // Top-k in registers needs every one of the k-th largest lane maxima.
  const bool res_topk = !greedy && use_k && top_k <= std::min<int64_t>(nvec, SNT);
  // The nucleus alone in registers: bfloat16 rows (128 keys per binade; a
  // float16 row's keys from the cut's lower bound up rarely fit the counts).
  const bool res_topp = !greedy && !use_k && use_p && logits_dtype == RRL_BF16;
  if (logits_dtype != RRL_F32 && (greedy || (!use_k && !use_p) || res_topk || res_topp) &&
      V % 8 == 0 && nvec <= (int64_t)SNT * RES_MAX_SLABS && ((uintptr_t)logits & 15u) == 0 &&
      (B == 1 || row_stride % 8 == 0)) {
    const int nslab = (int)((nvec + SNT - 1) / SNT);
    if (res_topp) {
      // Rows past the nucleus path's counts are left with token -1 for a
      // fill-in launch of the streaming kernel (its other workgroups return).
      const int rc = launch_sample_blocks<TagBF16, true>(a, nslab, st);
      if (rc != RRL_OK) return rc;
      SampleArgs f = a;
      f.fill_in = 1;
      return launch_sample<TagBF16>(f, st);
    }
    if (!res_topk)
      return logits_dtype == RRL_BF16 ? launch_sample_blocks<TagBF16, false>(a, nslab, st)
                                      : launch_sample_blocks<TagF16, false>(a, nslab, st);
    // A row whose candidate list overflows takes the streaming path inside
    // the same launch.
    return logits_dtype == RRL_BF16 ? launch_sample_resident<TagBF16>(a, nslab, st)
                                    : launch_sample_resident<TagF16>(a, nslab, st);
  }
  switch (logits_dtype) {
    case RRL_BF16: return launch_sample<TagBF16>(a, st);
    case RRL_F16: return launch_sample<TagF16>(a, st);
    default: return launch_sample<TagF32>(a, st);
  }
}
