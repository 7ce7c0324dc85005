// Fused LM head + token log-probs on the gfx950 matrix cores (MFMA), without
// the [tokens, vocabulary] logits tensor.
//
// The reference forms logits = hidden @ W^T (rosetrainer/model.py:499,641,
// rosetrainer/qwen3.py:508,556; no bias) and then log_softmax + gather
// (roserlhf/losses.py:14-38), keeping both [N, V] tensors and their gradient.
// With p = softmax(hidden_n W^T) and g_n = d loss / d logp_n the gradients are
//   dhidden_n = g_n (W[a_n] - sum_v p_nv W_v)        (a_n: the token's target)
//   dW_v      = sum_n g_n ([v == a_n] - p_nv) hidden_n
// The first sum is an attention-shaped product (queries = hidden, keys =
// values = W rows), so one streaming pass over the vocabulary computes it
// together with the log-sum-exp (online softmax, flash-attention style).  The
// second needs the final log-sum-exp: a mirrored pass streams the tokens past
// a stationary block of W rows and recomputes each logits tile.  Logits exist
// only as 32 x 64 tiles in registers and LDS.
//
// One kernel template serves both passes.  A workgroup (4 waves, one per SIMD)
// holds BM = 64 "stationary" rows X (tokens in the forward, vocabulary rows in
// the dW pass) and streams BN = 32-row tiles of Y (vocabulary rows, tokens).
// Wave w owns the hidden slice d in [w H/4, (w+1) H/4):
//   S phase:  S^T_w = Y[:, slice] X[:, slice]^T   (32 x 64 partial, MFMA
//             16x16x32 with the X fragments held in registers for the whole
//             pass and Y fragments read from LDS);
//   exchange: the four partials are summed through LDS; wave w finishes the
//             16 stationary rows of block w (softmax or gradient weights) and
//             publishes them as bf16/f16 MFMA A fragments;
//   acc phase: ACC_w[64 x slice] += P[64 x 32] Y[32 x slice], the Y tile read
//             transposed from LDS with ds_read_tr16_b64.
// The MFMA output layout of S^T (rows = tile rows) is already the A-fragment
// layout of the accumulation product once its k index is taken as
// {4g..4g+3, 16+4g..16+4g+3} for lane group g; the Y fragments of the
// accumulation product use the same k order.
//
// LDS (H = 1024): two Y tiles of 32 x 1024 (double buffer, 130 KB with rows
// padded so that both the natural and the transposed reads are bank-conflict
// free), 24 KB of partials, 4 KB of fragments, 1 KB of token records.
#include <mutex>
#include <type_traits>

#include "rrl_common.hpp"
#include "wave_common.hpp"

namespace rrl {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

constexpr int kBM = 64;   // stationary rows per workgroup
constexpr int kBN = 32;   // streamed rows per tile
constexpr int kNT = 256;  // four waves
constexpr float kLn2 = 0.69314718055994531f;
// Reference point of the forward's exponentials.  Row n's weights are
// exp(s - m_n) with m_n fixed at its first finite tile maximum plus
// kRefMargin, so the accumulators never need rescaling: values from
// kRefMargin + 63 below that maximum (negligible next to it) up to
// kRefHeadroom above it stay inside the float32 / bf16 exponent range.  A row
// whose logits rise further raises RRL_FLAG_LM_RANGE, and the caller reruns
// it with the reference taken from an exact log-sum-exp pass (mref_in).
constexpr float kRefMargin = 24.0f;
constexpr float kRefHeadroom = 88.0f;

enum { kModeFwd = 0, kModeFwdLseOnly = 1, kModeDw = 2 };

struct TagBF16 {};
struct TagF16 {};

template <class Tag>
__device__ __forceinline__ f32x4_t mfma(u32x4 a, u32x4 b, f32x4_t c) {
  if constexpr (std::is_same<Tag, TagBF16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Two floats to one packed 16-bit pair (round to nearest even).
template <class Tag>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (std::is_same<Tag, TagBF16>::value) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    f16x2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
}

template <class Tag>
__device__ __forceinline__ float widen(uint16_t h) {
  if constexpr (std::is_same<Tag, TagBF16>::value) return __uint_as_float((uint32_t)h << 16);
  else return (float)__builtin_bit_cast(_Float16, h);
}

// Tile rows in LDS are 2H + 32 bytes apart.  Both read patterns of the tile
// (natural: 16 lanes on 16 consecutive rows, one 16-byte chunk each;
// transposed: ds_read_b64_tr_b16 over 4 consecutive rows x 32 bytes) are
// bank-conflict free at that pitch for H = 1024 (measured with the
// SQ_LDS_BANK_CONFLICT counter on gfx950: zero at 2H + 32, two extra cycles
// per transposed read at 2H + 16, 2H + 48 and 2H + 64).  Every address is a
// per-lane base plus a compile-time offset.
constexpr int kRowPad = 32;

__device__ __forceinline__ u32x4 lds_load16(const uint8_t* base, uint32_t off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}
__device__ __forceinline__ void lds_store16(uint8_t* base, uint32_t off, u32x4 v) {
  *reinterpret_cast<u32x4*>(base + off) = v;
}
__device__ __forceinline__ uint2 lds_tr16(const uint8_t* base, uint32_t off) {
  const i16x4_t v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(const_cast<uint8_t*>(base + off)));
  return __builtin_bit_cast(uint2, v);
}

// The dW pass's token records of tile columns 4g + {0..3} and 16 + 4g + {0..3}
// (lane group g; `base` = the tile's records + 64 g bytes), with the wait for
// them.  The compiler models a 16-byte LDS-DMA load as a 4-byte store, and its
// alias analysis cannot place these reads apart from the next tile's loads
// still in flight into the other buffer: written as plain loads they get a
// vmcnt(0) wait, which would wait for the whole next tile.
__device__ __forceinline__ void lds_read_records(const uint8_t* base, f32x4_t (&r)[8]) {
  const uint32_t addr = (uint32_t)reinterpret_cast<uintptr_t>(base);
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %8 offset:16\n\t"
      "ds_read_b128 %2, %8 offset:32\n\t"
      "ds_read_b128 %3, %8 offset:48\n\t"
      "ds_read_b128 %4, %8 offset:256\n\t"
      "ds_read_b128 %5, %8 offset:272\n\t"
      "ds_read_b128 %6, %8 offset:288\n\t"
      "ds_read_b128 %7, %8 offset:304\n\t"
      "s_waitcnt lgkmcnt(0)"
      // early-clobber outputs: the address must outlive the first read
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]),
        "=&v"(r[6]), "=&v"(r[7])
      : "v"(addr)
      : "memory");
}

// Row exchange between the four 16-lane groups (lanes c, c+16, c+32, c+48).
__device__ __forceinline__ float xor16(float v) { return __shfl_xor(v, 16, 64); }
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// lse and logp of one row from its merged state: l = the sum of exp(s - mr)
// over its non-target columns, xt = the target column's logit (-inf: not
// seen), tg < 0: no target (logp 0).  lse = log(l e^mr + e^xt); logp = xt - lse
// is formed as -log1p(l e^(mr - xt)) so that it keeps its relative precision
// as p_target -> 1.
__device__ __forceinline__ void finish_row(float mr, float l, float xt, int32_t tg, float& lse,
                                           float& logp) {
  if (xt == -__builtin_huge_valf()) {
    lse = mr == -__builtin_huge_valf() ? -__builtin_huge_valf() : mr + logf(l);
    logp = tg < 0 ? 0.f : -__builtin_huge_valf();  // no target: 0
  } else if (mr == -__builtin_huge_valf() || l == 0.f) {
    lse = xt;
    logp = 0.f;
  } else {
    const float M = fmaxf(mr, xt);
    lse = M + logf(l * expf(mr - M) + expf(xt - M));
    const float d = mr - xt;
    const float z = l * expf(fminf(d, 80.f));
    logp = (d < 80.f && z < 1e30f) ? -log1pf(z) : -(d + logf(l));
  }
}

struct LmArgs {
  const void* x;  // stationary rows [nx, H], row stride x_ld elements
  int64_t x_ld;
  int32_t nx;
  const void* y;  // streamed rows [ny, H], row stride y_ld elements
  int64_t y_ld;
  int32_t ny;
  int32_t V;             // vocabulary size
  const int32_t* tgt;    // forward: target of each stationary row (token), -1 = none
  float* lse_out;        // forward: [nx]
  float* logp_out;       // forward: [nx]
  float* obar;           // forward: sum_{v != a} p_v W_v per token, [nx, H] (ld obar_ld)
  int64_t obar_ld;
  const float* mref_in;  // forward: per-token reference point (NULL: first-tile rule)
  const uint8_t* need_obar;  // forward: per token 1 = obar needed, 0 = log-prob only,
                             // 2 = neither (NULL: obar for every token)
  const int32_t* block_order;  // forward with need_obar: the 64-token blocks, those that
                               // need obar first, then those that need log-probs only,
                               // then those needing neither
  const int32_t* block_count;  // forward with need_obar: [0] blocks that need obar,
                               // [1] blocks that need obar or log-probs
  const int32_t* tile_list;  // dW pass: indices of the streamed tiles to visit (NULL: all)
  const int32_t* tile_count; // dW pass: number of entries of tile_list
  const float4* trec;    // dW pass: per streamed token {target bits, g, lse*log2e, g*(-expm1(logp))}
  void* dw;              // dW pass: [nx, H] (ld dw_ld), float32 or 16-bit
  int64_t dw_ld;
  int32_t dw_f32;
  int32_t dw_full;       // dW pass: workgroups that take a whole 64-row block
  int32_t dw_split;      // dW pass: parts each later block is split into (tile ranges)
  float* dw_part;        // dW pass: float32 [parts][64][H] partial rows of the split blocks
  int32_t* status;
};

template <int H>
struct LdsLayout {
  static constexpr int kRowBytes = H * 2 + kRowPad;
  static constexpr int kTileBytes = kBN * kRowBytes;
  static constexpr int kFragOff = 2 * kTileBytes;                 // [4 blocks][64] x 16 B
  static constexpr int kPartOff = kFragOff + 4 * 64 * 16;          // [12 slots][2][64] x 16 B
  static constexpr int kRecOff = kPartOff + 12 * 2 * 64 * 16;      // [2][32] x 16 B (dW pass)
  static constexpr int kAlphaOff = kPartOff;                       // [64] floats (epilogue only)
  static constexpr int kTotal = kRecOff + 2 * kBN * 16;
  static_assert(kTotal <= 160 * 1024, "LDS budget of one workgroup");
};

template <class Tag, int MODE, int H>
__device__ __forceinline__ void lm_tile_body(const LmArgs& a, uint8_t* lds, const int32_t x0,
                                             const int32_t t_lo, const int32_t t_hi,
                                             float* const part_out) {
  constexpr int DW = H / 4;                 // hidden slice of each wave (S depth and accumulator)
  constexpr int KQ = DW / 32;               // k-steps of the S product over one slice
  constexpr int DB = DW / 16;               // 16-column blocks of the accumulator per wave
  constexpr int CH = H / 8;                 // 16-byte chunks per row
  constexpr bool kAcc = MODE != kModeFwdLseOnly;
  using L = LdsLayout<H>;
  static_assert(H % 128 == 0 && H <= 1024, "hidden size must be a multiple of 128, at most 1024");

  const int tid = threadIdx.x, lane = tid & 63, lg = lane >> 4, lc = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int dw0 = w * DW;

  // ---- stationary fragments of all 64 rows over this wave's hidden slice,
  // row blocks rotated so that slot 0 is the wave's own block:
  // xs[j][ks] = X[x0 + 16((w + j) mod 4) + lc][dw0 + 32ks + 8lg .. +7] ----
  u32x4 xs[4][KQ];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int32_t row = x0 + 16 * ((w + j) & 3) + lc;
    const uint16_t* p = static_cast<const uint16_t*>(a.x) + (int64_t)row * a.x_ld + dw0 + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < KQ; ++ks)
      xs[j][ks] = row < a.nx ? *reinterpret_cast<const u32x4*>(p + 32 * ks) : u32x4{0, 0, 0, 0};
  }

  f32x4_t acc[4][kAcc ? DB : 1];
  if constexpr (kAcc) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[nb][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Forward row state of stationary row x0 + 16w + lc (replicated over lg).
  const int32_t my_row = x0 + 16 * w + lc;
  int32_t tg = -1;
  if constexpr (MODE != kModeDw) {
    if (my_row < a.nx) {
      tg = a.tgt[my_row];
      if (tg >= a.V) {  // a negative id is "no target" (cross-entropy's ignore_index)
        raise_flag(a.status, RRL_FLAG_TARGET_RANGE);
        tg = -1;
      }
    }
  }
  float m_ref = -__builtin_huge_valf(), l_part = 0.f, xa = -__builtin_huge_valf();
  if constexpr (MODE == kModeFwd) {
    if (a.mref_in != nullptr && my_row < a.nx) m_ref = a.mref_in[my_row];
  }

  // Streamed tiles t_lo .. t_hi - 1 (of tile_list when given).
  // Index of tile t (tile_list read one tile ahead of its use: the wait for
  // the read is then the end-of-tile wait that precedes it).
  auto tile_index = [&](int32_t t) { return a.tile_list ? a.tile_list[t] : t; };

  // ---- tile loads, global -> LDS directly (buffer loads with the LDS bit:
  // no registers).  One wave-wide load writes 64 consecutive lanes x UNIT
  // bytes of LDS, so a row (2H bytes, padded rows) is PER_ROW loads; UNIT is
  // 16 bytes when a row is whole kilobytes, else 4.  Each wave issues WLOADS
  // of them per tile, spread over the S phase's k-steps (CHUNK per step): a
  // wave that issued them all at once would stall on the full load queue
  // before its first MFMA.  The caller waits for vmcnt(0) before the barrier
  // that publishes the tile. ----
  constexpr int UNIT = (2 * H) % 1024 == 0 ? 16 : 4;
  constexpr int PER_ROW = 2 * H / (64 * UNIT);
  constexpr int WLOADS = kBN * PER_ROW / 4;  // per wave per tile
  static_assert(kBN * PER_ROW % 4 == 0, "tile load split");
  typedef __attribute__((address_space(3))) void lds_void_t;
  // dW pass: the 32 token records of the next tile go through registers of
  // wave 0's first 32 lanes (a plain load issued ahead of the tile's loads)
  // and are written to LDS at the end of the current tile.
  float4 rec_next = make_float4(0.f, 0.f, 0.f, 0.f);
  constexpr int CHUNK = (WLOADS + KQ - 1) / KQ;
  // Descriptor of the tile starting at streamed row r0 (and, in the dW pass,
  // the load of its token records).
  auto tile_src = [&](int32_t r0) {
    const int32_t rows = a.ny - r0 < kBN ? a.ny - r0 : kBN;
    if constexpr (MODE == kModeDw) {
      // records past the last token read as zeros (g = 0)
      if (w == 0 && lane < kBN)
        rec_next = lane < rows ? a.trec[r0 + lane] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const uint16_t* base = static_cast<const uint16_t*>(a.y) + (int64_t)r0 * a.y_ld;
    // Rows at or past `rows` start at or beyond the descriptor's byte count
    // (row stride >= H), so they read as zeros.
    return row_rsrc(base, (uint32_t)(((rows - 1) * a.y_ld + H) * 2));
  };
  // This wave's loads i0 .. i1-1 of a tile into buffer tb (i0, i1 constant
  // after unrolling).
  auto issue_loads = [&](const __amdgpu_buffer_rsrc_t& rs, uint8_t* tb, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      const int q = w * WLOADS + i;  // wave-uniform
      const int j = q / PER_ROW, part = q % PER_ROW;
      const uint32_t goff = (uint32_t)(j * a.y_ld * 2 + part * 64 * UNIT + lane * UNIT);
      lds_void_t* dst = (lds_void_t*)(tb + j * L::kRowBytes + part * 64 * UNIT);
      if constexpr (UNIT == 16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, goff, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 4, goff, 0, 0, 0);
    }
  };
  auto publish_records = [&](int buf) {
    if constexpr (MODE == kModeDw) {
      if (w == 0 && lane < kBN)
        *reinterpret_cast<float4*>(lds + L::kRecOff + buf * kBN * 16 + lane * 16) = rec_next;
    }
  };

  int32_t r0_next = t_lo < t_hi ? __builtin_amdgcn_readfirstlane(tile_index(t_lo) * kBN) : 0;
  int32_t idx_ahead = t_lo + 1 < t_hi ? tile_index(t_lo + 1) : 0;
  if (t_lo < t_hi) issue_loads(tile_src(r0_next), lds, 0, WLOADS);
  // Every prologue load (the stationary fragments and tile 0) has landed.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt, lgkmcnt untouched
  publish_records(0);
  lds_barrier();

  uint8_t* const frag = lds + L::kFragOff;
  float* const alpha = reinterpret_cast<float*>(lds + L::kAlphaOff);

  // One tile: tb is the tile being computed on, tn the buffer its successor
  // is loaded into.  The two are distinct LDS objects for the compiler
  // (restrict): without that, its alias analysis cannot tell the transposed
  // reads of tb from the in-flight loads into tn and waits for all of them
  // (vmcnt(0)) before the first transposed read.
  auto tile_step = [&](const uint8_t* __restrict__ tb, uint8_t* __restrict__ tn, const int buf,
                       const int32_t t) __attribute__((always_inline)) {
    // Tile t+1 goes to the other buffer, free since barrier C of tile t-1;
    // it has this whole tile's work to land.
    const bool more = t + 1 < t_hi;
    const int32_t r0 = r0_next;
    __amdgpu_buffer_rsrc_t rs_next;
    if (more) {
      r0_next = __builtin_amdgcn_readfirstlane(idx_ahead * kBN);
      rs_next = tile_src(r0_next);
      if (t + 2 < t_hi) idx_ahead = tile_index(t + 2);
    }

    // ---- S phase: partial S^T[32 x 64] of the tile against all 64 rows over
    // this wave's hidden slice; each tile fragment read from LDS feeds four
    // MFMAs (one per 16-row block).  The fragments of step ks+2 are read while
    // step ks's MFMAs run (the scheduling fences keep the compiler from
    // hoisting every read). ----
    f32x4_t tot[2];
    {
      f32x4_t sa[4][2];
#pragma unroll
      for (int j = 0; j < 4; ++j) sa[j][0] = sa[j][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const uint8_t* abase = tb + lc * L::kRowBytes + 2 * dw0 + 16 * lg;
      auto af_at = [&](int ks, int vb) {
        return lds_load16(abase, 64 * ks + vb * 16 * L::kRowBytes);
      };
      u32x4 af[3][2];
      af[0][0] = af_at(0, 0);
      af[0][1] = af_at(0, 1);
      if (KQ > 1) {
        af[1][0] = af_at(1, 0);
        af[1][1] = af_at(1, 1);
      }
#pragma unroll
      for (int ks = 0; ks < KQ; ++ks) {
        if (more && ks * CHUNK < WLOADS)
          issue_loads(rs_next, tn, ks * CHUNK,
                      ks * CHUNK + CHUNK < WLOADS ? ks * CHUNK + CHUNK : WLOADS);
        if (ks + 2 < KQ) {
          af[(ks + 2) % 3][0] = af_at(ks + 2, 0);
          af[(ks + 2) % 3][1] = af_at(ks + 2, 1);
        }
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            sa[j][vb] = mfma<Tag>(af[ks % 3][vb], xs[j][ks], sa[j][vb]);
        __builtin_amdgcn_sched_barrier(0);
      }

      // ---- exchange: wave w sends its partials of the other three row blocks
      // to their owners (slot 3d + s' holds source s' of the other sources
      // of destination block d, in source order), then adds them to its own
      // partial in that order. ----
      uint8_t* const part = lds + L::kPartOff;
#pragma unroll
      for (int j = 1; j < 4; ++j) {
        const int d = (w + j) & 3;  // wave-uniform
        const int sl = 3 * d + (w < d ? w : w - 1);
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
          lds_store16(part, (uint32_t)((2 * sl + vb) * 1024 + lane * 16),
                      __builtin_bit_cast(u32x4, sa[j][vb]));
      }
      lds_barrier();  // A: partials published
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) {
        f32x4_t o[3];
#pragma unroll
        for (int q = 0; q < 3; ++q)
          o[q] = __builtin_bit_cast(
              f32x4_t, lds_load16(part, (uint32_t)((2 * (3 * w + q) + vb) * 1024 + lane * 16)));
        tot[vb] = ((sa[0][vb] + o[0]) + o[1]) + o[2];
      }
    }

    // ---- this wave's 16 rows: softmax weights or gradient weights ----
    float s[8];
    {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[r] = tot[0][r];
        s[4 + r] = tot[1][r];
      }
    }
    // Tile column of value i: 4lg + (i & 3) + 16 (i >> 2).
    uint32_t pk[4] = {0u, 0u, 0u, 0u};
    if constexpr (MODE == kModeDw) {
      // P^T[v][n] = g_n ([v == a_n] - exp(s - lse_n)), the target entry as
      // g_n (-expm1(logp_n)) (exact as p -> 1).
      f32x4_t rcs[8];
      lds_read_records(lds + L::kRecOff + buf * kBN * 16 + 64 * lg, rcs);
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const f32x4_t rc = rcs[i];
        const int32_t an = __float_as_int(rc.x);
        const float gn = rc.y;
        const float e = exp2_hw(s[i] * kLog2e - rc.z);
        p[i] = gn == 0.f ? 0.f : (an == (int32_t)my_row ? rc.w : -gn * e);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) pk[i] = pack2<Tag>(p[2 * i], p[2 * i + 1]);
    } else {
      // Softmax weights of row my_row over this tile (target column held out).
      // Columns past the vocabulary (last tile only) and a row's target column
      // (in a tile holding some row's target) take the per-column path; the
      // test is wave-uniform.
      const bool tgt_here = tg >= r0 && tg < r0 + kBN;
      if (r0 + kBN > a.V || __builtin_amdgcn_ballot_w64(tgt_here) != 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int32_t v = r0 + 4 * lg + (i & 3) + 16 * (i >> 2);
          if (v >= a.V) s[i] = -__builtin_huge_valf();
          if (v == tg) {
            xa = s[i];
            s[i] = -__builtin_huge_valf();
          }
        }
      }
      float tmax = -__builtin_huge_valf();
#pragma unroll
      for (int i = 0; i < 8; ++i) tmax = fmaxf(tmax, s[i]);
      if constexpr (MODE == kModeFwdLseOnly) {
        // No accumulator: each lane keeps an exact running maximum of its own
        // columns, l rescaled as it moves; the row's four lanes merge at the end.
        if (tmax > m_ref) {
          l_part *= m_ref == -__builtin_huge_valf() ? 0.f : exp2_hw((m_ref - tmax) * kLog2e);
          m_ref = tmax;
        }
      } else {
        // The row's reference point, the same in its four lanes, is set once
        // from its first finite tile maximum and then stays fixed (no
        // accumulator rescaling): the cross-lane maximum runs only while some
        // row of the wave has none yet.
        if (__builtin_amdgcn_ballot_w64(m_ref == -__builtin_huge_valf()) != 0) {
          float rmax = fmaxf(tmax, xor16(tmax));
          rmax = fmaxf(rmax, xor32(rmax));
          if (m_ref == -__builtin_huge_valf() && rmax > -__builtin_huge_valf())
            m_ref = rmax + kRefMargin;
        }
        if (tmax > m_ref + (kRefHeadroom - kRefMargin) && my_row < a.nx)
          raise_flag(a.status, RRL_FLAG_LM_RANGE);
      }
      const float mb = m_ref == -__builtin_huge_valf() ? 0.f : m_ref * kLog2e;
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = exp2_hw(s[i] * kLog2e - mb);  // exp(-inf) = 0
        l_part += p[i];
      }
      if constexpr (kAcc) {
#pragma unroll
        for (int i = 0; i < 4; ++i) pk[i] = pack2<Tag>(p[2 * i], p[2 * i + 1]);
      }
    }
    if constexpr (kAcc) {
      lds_store16(frag, (w * 64 + lane) * 16, u32x4{pk[0], pk[1], pk[2], pk[3]});
      lds_barrier();  // B: every wave's fragments published

      u32x4 pf[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) pf[nb] = lds_load16(frag, (nb * 64 + lane) * 16);
      // ---- acc phase: ACC_w[64 x DW] += P[64 x 32] Y[32 x DW] ----
      // B fragment of block db: Y[k][dw0 + 16db + lc] for k = 4lg + e and
      // 16 + 4lg + e, two transposing reads; block db+1 is read while the
      // MFMAs of db run.
      const uint8_t* bbase =
          tb + (4 * lg + (lc >> 2)) * L::kRowBytes + (dw0 + 4 * (lc & 3)) * 2;
      auto bf_at = [&](int db) {
        const uint2 b1 = lds_tr16(bbase, 32 * db);
        const uint2 b2 = lds_tr16(bbase, 32 * db + 16 * L::kRowBytes);
        return u32x4{b1.x, b1.y, b2.x, b2.y};
      };
      u32x4 bf[3];
      bf[0] = bf_at(0);
      if (DB > 1) bf[1] = bf_at(1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        if (db + 2 < DB) bf[(db + 2) % 3] = bf_at(db + 2);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[nb][db] = mfma<Tag>(pf[nb], bf[db % 3], acc[nb][db]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of tile t+1 landed
    if (more) publish_records(buf ^ 1);  // tile t's records were read before barrier B
    lds_barrier();  // C: tile t+1 complete; tile t's reads done
  };
  for (int32_t t = t_lo; t < t_hi; ++t) {
    const int buf = (int)((t - t_lo) & 1);
    tile_step(lds + buf * L::kTileBytes, lds + (buf ^ 1) * L::kTileBytes, buf, t);
  }

  // ---- epilogue ----
  if constexpr (MODE != kModeDw) {
    if constexpr (MODE == kModeFwdLseOnly) {
      // merge the four lanes' running maxima of each row
      float M = fmaxf(m_ref, xor16(m_ref));
      M = fmaxf(M, xor32(M));
      l_part = m_ref == M ? l_part : l_part * exp2_hw((m_ref - M) * kLog2e);
      m_ref = M;
    }
    float l = l_part + xor16(l_part);
    l += xor32(l);
    float xt = fmaxf(xa, xor16(xa));
    xt = fmaxf(xt, xor32(xt));
    float lse, logp;
    const float mr = m_ref;
    finish_row(mr, l, xt, tg, lse, logp);
    if (lg == 0 && my_row < a.nx) {
      a.lse_out[my_row] = lse;
      a.logp_out[my_row] = logp;
    }
    if constexpr (MODE == kModeFwd) {
      // Obar = acc * exp(m_ref - lse): every wave scales all 64 rows.
      if (lg == 0) alpha[16 * w + lc] = mr == -__builtin_huge_valf() ? 0.f : expf(mr - lse);
      lds_barrier();
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const f32x4_t sc = *reinterpret_cast<const f32x4_t*>(alpha + 16 * nb + 4 * lg);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int32_t row = x0 + 16 * nb + 4 * lg + r;
          if (row >= a.nx) continue;
          float* o = a.obar + (int64_t)row * a.obar_ld + dw0 + lc;
#pragma unroll
          for (int db = 0; db < DB; ++db) o[16 * db] = acc[nb][db][r] * sc[r];
        }
      }
    }
  } else {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t row = x0 + 16 * nb + 4 * lg + r;
        if (row >= a.nx) continue;
        if (part_out != nullptr) {  // a part of a split block: float32 partial rows
          float* o = part_out + (int64_t)(16 * nb + 4 * lg + r) * H + dw0 + lc;
#pragma unroll
          for (int db = 0; db < DB; ++db) o[16 * db] = acc[nb][db][r];
        } else if (a.dw_f32) {
          float* o = static_cast<float*>(a.dw) + (int64_t)row * a.dw_ld + dw0 + lc;
#pragma unroll
          for (int db = 0; db < DB; ++db) o[16 * db] = acc[nb][db][r];
        } else {
          uint16_t* o = static_cast<uint16_t*>(a.dw) + (int64_t)row * a.dw_ld + dw0 + lc;
#pragma unroll
          for (int db = 0; db < DB; ++db)
            o[16 * db] = (uint16_t)(pack2<Tag>(acc[nb][db][r], 0.f) & 0xFFFFu);
        }
      }
    }
  }
}

template <class Tag, int H>
__device__ __forceinline__ void lm_lse_body(const LmArgs& a, uint8_t* lds, const int32_t x_a,
                                            const int32_t x_b);

template <class Tag, int MODE, int H>
__global__ __launch_bounds__(kNT, 1) void lm_tile_kernel(LmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[LdsLayout<H>::kTotal];
  if constexpr (MODE == kModeFwd) {
    // With need_obar the launch covers every 64-token block, in block_order:
    // workgroup i < count takes block block_order[i], which needs obar; the
    // following workgroups take the remaining blocks two at a time, through
    // the log-sum-exp pass when some token of the block needs its log-prob,
    // else writing 0 as every token's lse and log-prob (need value 2 on all
    // 64: no work); surplus workgroups return at once.
    // Listing the obar blocks first, rather than taking blocks in token
    // order, spreads them evenly over the eight XCDs (consecutive workgroups
    // go to the XCDs in turn): masks that end each sequence in a run of
    // masked blocks otherwise load some XCDs with most of the obar work
    // (measured: as slow as obar for every block).  One launch rather than
    // two lets the log-sum-exp workgroups fill the obar pass's last round.
    if (a.block_order != nullptr) {
      const int32_t count = *a.block_count, i = (int32_t)blockIdx.x;
      if (i < count) {
        const int32_t blk = __builtin_amdgcn_readfirstlane(a.block_order[i]);
        lm_tile_body<Tag, MODE, H>(a, lds, blk * kBM, 0, (a.ny + kBN - 1) / kBN, nullptr);
        return;
      }
      const int32_t nblocks = (a.nx + kBM - 1) / kBM, live = a.block_count[1];
      const int32_t e = count + 2 * (i - count);
      if (e >= nblocks) return;
      // Blocks of this pair that need no output: zeros, one thread per token.
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (e + q >= live && e + q < nblocks && threadIdx.x < kBM) {
          const int32_t row = a.block_order[e + q] * kBM + (int32_t)threadIdx.x;
          if (row < a.nx) {
            a.lse_out[row] = 0.f;
            a.logp_out[row] = 0.f;
          }
        }
      }
      if (e >= live) return;
      const int32_t x_a = __builtin_amdgcn_readfirstlane(a.block_order[e]) * kBM;
      const int32_t x_b =
          e + 1 < live ? __builtin_amdgcn_readfirstlane(a.block_order[e + 1]) * kBM : -1;
      lm_lse_body<Tag, H>(a, lds, x_a, x_b);
      return;
    }
  }
  if constexpr (MODE == kModeDw) {
    // Blocks past dw_full are split into dw_split ranges of the tile list
    // (the last, partial round of workgroups then has dw_split times as many,
    // each with 1 / dw_split of the work); their float32 partial rows are
    // summed by lm_dw_reduce_kernel.
    const int32_t nt = a.tile_count ? *a.tile_count : (a.ny + kBN - 1) / kBN;
    const int32_t i = (int32_t)blockIdx.x;
    if (i < a.dw_full) {
      lm_tile_body<Tag, MODE, H>(a, lds, i * kBM, 0, nt, nullptr);
    } else {
      const int32_t j = i - a.dw_full, part = j % a.dw_split;
      const int32_t lo = (int32_t)((int64_t)part * nt / a.dw_split);
      const int32_t hi = (int32_t)((int64_t)(part + 1) * nt / a.dw_split);
      lm_tile_body<Tag, MODE, H>(a, lds, (a.dw_full + j / a.dw_split) * kBM, lo, hi,
                                 a.dw_part + (int64_t)j * kBM * H);
    }
    return;
  }
  lm_tile_body<Tag, MODE, H>(a, lds, (int32_t)blockIdx.x * kBM, 0, (a.ny + kBN - 1) / kBN,
                             nullptr);
}

// ---- log-sum-exp-only pass (no obar), 128 stationary rows per workgroup ----
// Without the accumulator a wave has the registers for 32 rows over the whole
// hidden size (xs: 256 registers, in the accumulation registers), so the
// score product needs no cross-wave exchange and each tile fetched from L2
// serves twice the rows of the obar pass.  Wave w holds rows
// xb + 32 (w & 1) + [0, 32) of block xb = (w < 2 ? x_a : x_b) (x_b < 0: none).
template <class Tag, int H>
__device__ __forceinline__ void lm_lse_body(const LmArgs& a, uint8_t* lds, const int32_t x_a,
                                            const int32_t x_b) {
  constexpr int KF = H / 32;  // k-steps over the whole hidden size
  using L = LdsLayout<H>;
  static_assert(H % 128 == 0 && H <= 1024, "hidden size must be a multiple of 128, at most 1024");

  const int tid = threadIdx.x, lane = tid & 63, lg = lane >> 4, lc = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int32_t xb = w < 2 ? x_a : x_b;
  int32_t row[2];
  bool ok[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    row[rb] = xb + 32 * (w & 1) + 16 * rb + lc;
    ok[rb] = xb >= 0 && row[rb] < a.nx;
  }
  u32x4 xs[2][KF];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const uint16_t* p =
        static_cast<const uint16_t*>(a.x) + (int64_t)(ok[rb] ? row[rb] : 0) * a.x_ld + 8 * lg;
#pragma unroll
    for (int ks = 0; ks < KF; ++ks)
      xs[rb][ks] = ok[rb] ? *reinterpret_cast<const u32x4*>(p + 32 * ks) : u32x4{0, 0, 0, 0};
  }
  int32_t tg[2];
  float m[2], l[2], xa[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    tg[rb] = -1;
    if (ok[rb]) {
      tg[rb] = a.tgt[row[rb]];
      if (tg[rb] >= a.V) {
        raise_flag(a.status, RRL_FLAG_TARGET_RANGE);
        tg[rb] = -1;
      }
    }
    m[rb] = -__builtin_huge_valf();
    l[rb] = 0.f;
    xa[rb] = -__builtin_huge_valf();
  }

  const int32_t ntiles = (a.ny + kBN - 1) / kBN;
  constexpr int UNIT = (2 * H) % 1024 == 0 ? 16 : 4;
  constexpr int PER_ROW = 2 * H / (64 * UNIT);
  constexpr int WLOADS = kBN * PER_ROW / 4;
  constexpr int CHUNK = (WLOADS + KF - 1) / KF;
  typedef __attribute__((address_space(3))) void lds_void_t;
  auto tile_src = [&](int32_t r0) {
    const int32_t rows = a.ny - r0 < kBN ? a.ny - r0 : kBN;
    const uint16_t* base = static_cast<const uint16_t*>(a.y) + (int64_t)r0 * a.y_ld;
    return row_rsrc(base, (uint32_t)(((rows - 1) * a.y_ld + H) * 2));
  };
  auto issue_loads = [&](const __amdgpu_buffer_rsrc_t& rs, uint8_t* tb, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      const int q = w * WLOADS + i;
      const int j = q / PER_ROW, part = q % PER_ROW;
      const uint32_t goff = (uint32_t)(j * a.y_ld * 2 + part * 64 * UNIT + lane * UNIT);
      lds_void_t* dst = (lds_void_t*)(tb + j * L::kRowBytes + part * 64 * UNIT);
      if constexpr (UNIT == 16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, goff, 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 4, goff, 0, 0, 0);
    }
  };
  if (ntiles > 0) issue_loads(tile_src(0), lds, 0, WLOADS);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the prologue loads landed
  lds_barrier();

  auto tile_step = [&](const uint8_t* __restrict__ tb, uint8_t* __restrict__ tn,
                       const int32_t t) __attribute__((always_inline)) {
    const bool more = t + 1 < ntiles;
    const int32_t r0 = t * kBN;
    __amdgpu_buffer_rsrc_t rs_next;
    if (more) rs_next = tile_src(r0 + kBN);
    f32x4_t sa[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) sa[rb][0] = sa[rb][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint8_t* abase = tb + lc * L::kRowBytes + 16 * lg;
    auto af_at = [&](int ks, int vb) { return lds_load16(abase, 64 * ks + vb * 16 * L::kRowBytes); };
    u32x4 af[3][2];
    af[0][0] = af_at(0, 0);
    af[0][1] = af_at(0, 1);
    if (KF > 1) {
      af[1][0] = af_at(1, 0);
      af[1][1] = af_at(1, 1);
    }
#pragma unroll
    for (int ks = 0; ks < KF; ++ks) {
      if (more && ks * CHUNK < WLOADS)
        issue_loads(rs_next, tn, ks * CHUNK,
                    ks * CHUNK + CHUNK < WLOADS ? ks * CHUNK + CHUNK : WLOADS);
      if (ks + 2 < KF) {
        af[(ks + 2) % 3][0] = af_at(ks + 2, 0);
        af[(ks + 2) % 3][1] = af_at(ks + 2, 1);
      }
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          sa[rb][vb] = mfma<Tag>(af[ks % 3][vb], xs[rb][ks], sa[rb][vb]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Per row block: the target column held out, columns past the vocabulary
    // dropped (both on a wave-uniform slow path), then each lane's exact
    // running maximum and sum of its own columns (merged at the end).
    const bool slow = r0 + kBN > a.V ||
                      __builtin_amdgcn_ballot_w64((tg[0] >= r0 && tg[0] < r0 + kBN) ||
                                                  (tg[1] >= r0 && tg[1] < r0 + kBN)) != 0;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      float sv[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[r] = sa[rb][0][r];
        sv[4 + r] = sa[rb][1][r];
      }
      if (slow) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int32_t v = r0 + 4 * lg + (i & 3) + 16 * (i >> 2);
          if (v >= a.V) sv[i] = -__builtin_huge_valf();
          if (v == tg[rb]) {
            xa[rb] = sv[i];
            sv[i] = -__builtin_huge_valf();
          }
        }
      }
      float tmax = sv[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, sv[i]);
      if (tmax > m[rb]) {
        l[rb] *= m[rb] == -__builtin_huge_valf() ? 0.f : exp2_hw((m[rb] - tmax) * kLog2e);
        m[rb] = tmax;
      }
      const float mb = m[rb] == -__builtin_huge_valf() ? 0.f : m[rb] * kLog2e;
#pragma unroll
      for (int i = 0; i < 8; ++i) l[rb] += exp2_hw(sv[i] * kLog2e - mb);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of tile t+1 landed
    lds_barrier();                       // tile t+1 complete; tile t's reads done
  };
  for (int32_t t = 0; t < ntiles; ++t) {
    const int buf = (int)(t & 1);
    tile_step(lds + buf * L::kTileBytes, lds + (buf ^ 1) * L::kTileBytes, t);
  }

#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float M = fmaxf(m[rb], xor16(m[rb]));
    M = fmaxf(M, xor32(M));
    float lr = m[rb] == M ? l[rb] : l[rb] * exp2_hw((m[rb] - M) * kLog2e);
    lr += xor16(lr);
    lr += xor32(lr);
    float xt = fmaxf(xa[rb], xor16(xa[rb]));
    xt = fmaxf(xt, xor32(xt));
    float lse, logp;
    finish_row(M, lr, xt, tg[rb], lse, logp);
    if (lg == 0 && ok[rb]) {
      a.lse_out[row[rb]] = lse;
      a.logp_out[row[rb]] = logp;
    }
  }
}

template <class Tag, int H>
__global__ __launch_bounds__(kNT, 1) void lm_lse_kernel(LmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * LdsLayout<H>::kTileBytes];
  const int32_t x_a = (int32_t)blockIdx.x * 2 * kBM;
  lm_lse_body<Tag, H>(a, lds, x_a, x_a + kBM < a.nx ? x_a + kBM : -1);
}

// Tiles of 32 streamed tokens that hold a token with g != 0 (the others
// contribute exactly zero to dW): flags, then one workgroup lists them in
// ascending order.
__global__ __launch_bounds__(256) void lm_tile_flags_kernel(int32_t n, const float* g,
                                                            uint8_t* flags) {
  const int32_t ntiles = (n + kBN - 1) / kBN;
  for (int32_t tile = blockIdx.x * 256 + threadIdx.x; tile < ntiles;
       tile += gridDim.x * 256) {
    const int32_t b = tile * kBN, e = n - b < kBN ? n : b + kBN;
    bool act = false;
    if (e - b == kBN && ((uintptr_t)(g + b) & 15) == 0) {
      const float4* q = reinterpret_cast<const float4*>(g + b);
#pragma unroll
      for (int i = 0; i < kBN / 4; ++i) {
        const float4 v = q[i];
        act |= (v.x != 0.f) | (v.y != 0.f) | (v.z != 0.f) | (v.w != 0.f);
      }
    } else {
      for (int32_t i = b; i < e; ++i) act |= g[i] != 0.f;
    }
    flags[tile] = act ? 1 : 0;
  }
}

__global__ __launch_bounds__(1024) void lm_tile_list_kernel(int32_t n, const uint8_t* flags,
                                                            int32_t* list, int32_t* count) {
  __shared__ int32_t wcount[16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int32_t ntiles = (n + kBN - 1) / kBN;
  int32_t base = 0;
  for (int32_t c0 = 0; c0 < ntiles; c0 += 1024) {
    const int32_t tile = c0 + tid;
    const bool act = tile < ntiles && flags[tile] != 0;
    const uint64_t bal = __builtin_amdgcn_ballot_w64(act);
    if (lane == 0) wcount[wv] = __popcll(bal);
    __syncthreads();
    int32_t before = base, total = base;
    for (int k = 0; k < 16; ++k) {
      if (k < wv) before += wcount[k];
      total += wcount[k];
    }
    if (act) list[before + __popcll(bal & ((1ull << lane) - 1ull))] = tile;
    base = total;
    __syncthreads();
  }
  if (tid == 0) *count = base;
}

// Order of the forward's 64-token blocks (one workgroup): those with a token
// whose obar is needed (need value 1) first, then those with a token that
// needs its log-prob (value 0), then the rest (every token 2), each group in
// ascending order; order[nblocks] = the first group's size, order[nblocks +
// 1] = the first two groups' size.
__global__ __launch_bounds__(1024) void lm_block_order_kernel(int32_t n, const uint8_t* need,
                                                              int32_t* order) {
  __shared__ int32_t wcount[16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int32_t nblocks = (n + kBM - 1) / kBM;
  int32_t base = 0;
  for (int pass = 0; pass < 3; ++pass) {
    for (int32_t c0 = 0; c0 < nblocks; c0 += 1024) {
      const int32_t blk = c0 + tid;
      bool obar = false, live = false;  // a value 1; a value other than 2
      if (blk < nblocks) {
        const int32_t b = blk * kBM, e = n - b < kBM ? n : b + kBM;
        if (e - b == kBM && ((uintptr_t)(need + b) & 15) == 0) {
          const uint4* q = reinterpret_cast<const uint4*>(need + b);
#pragma unroll
          for (int i = 0; i < kBM / 16; ++i) {
            const uint4 v = q[i];
            obar |= ((v.x | v.y | v.z | v.w) & 0x01010101u) != 0u;
            live |= ((v.x ^ 0x02020202u) | (v.y ^ 0x02020202u) | (v.z ^ 0x02020202u) |
                     (v.w ^ 0x02020202u)) != 0u;
          }
        } else {
          for (int32_t i = b; i < e; ++i) {
            obar |= (need[i] & 1) != 0;
            live |= need[i] != 2;
          }
        }
      }
      const int grp = obar ? 0 : (live ? 1 : 2);
      const bool take = blk < nblocks && grp == pass;
      const uint64_t bal = __builtin_amdgcn_ballot_w64(take);
      if (lane == 0) wcount[wv] = __popcll(bal);
      __syncthreads();
      int32_t before = base, total = base;
      for (int k = 0; k < 16; ++k) {
        if (k < wv) before += wcount[k];
        total += wcount[k];
      }
      if (take) order[before + __popcll(bal & ((1ull << lane) - 1ull))] = blk;
      base = total;
      __syncthreads();
    }
    if (pass < 2 && tid == 0) order[nblocks + pass] = base;
  }
}

// Per-token records of the dW pass: {target (bits), g, lse*log2(e),
// g*(-expm1(logp))}; a token with no valid target gets target -1.
__global__ __launch_bounds__(256) void lm_token_records_kernel(int64_t n, int32_t V,
                                                               const int32_t* tgt,
                                                               const float* lse,
                                                               const float* logp,
                                                               const float* g, float4* out) {
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    const int32_t a = tgt[i];
    const bool ok = a >= 0 && a < V;
    // a token without a valid target has no gradient, whatever g holds
    const float gi = ok ? g[i] : 0.f;
    out[i] = make_float4(__int_as_float(ok ? a : -1), gi, lse[i] * kLog2e,
                         ok ? gi * -expm1f(logp[i]) : 0.f);
  }
}

// Rows of the split dW blocks (blocks full, full + 1, ...): dw[row] = the sum
// over the parts, in part order, of their float32 partial rows.
template <class Tag>
__global__ __launch_bounds__(256) void lm_dw_reduce_kernel(int32_t nrows, int32_t parts,
                                                           int32_t full, int32_t H, int32_t nx,
                                                           const float* part, void* dw,
                                                           int64_t dw_ld, int32_t dw_f32) {
  for (int32_t rr = blockIdx.x; rr < nrows; rr += gridDim.x) {
    const int32_t blk = rr / kBM, r = rr % kBM;
    const int32_t row = full * kBM + rr;
    if (row >= nx) continue;
    for (int32_t c = threadIdx.x; c < H; c += 256) {
      float v = 0.f;
      for (int32_t q = 0; q < parts; ++q)
        v += part[((int64_t)(blk * parts + q) * kBM + r) * H + c];
      if (dw_f32)
        static_cast<float*>(dw)[(int64_t)row * dw_ld + c] = v;
      else
        static_cast<uint16_t*>(dw)[(int64_t)row * dw_ld + c] =
            (uint16_t)(pack2<Tag>(v, 0.f) & 0xFFFFu);
    }
  }
}

// dhidden[n] = g_n ((-expm1(logp_n)) W[a_n] - obar_n), 16-bit out.
template <class Tag>
__global__ __launch_bounds__(256) void lm_dhidden_kernel(int64_t n, int32_t H, int32_t V,
                                                         const uint16_t* w, int64_t w_ld,
                                                         const int32_t* tgt, const float* logp,
                                                         const float* g, const float* obar,
                                                         int64_t obar_ld, uint16_t* dh,
                                                         int64_t dh_ld) {
  for (int64_t i = blockIdx.x; i < n; i += gridDim.x) {
    const int32_t a = tgt[i];
    const bool valid = a >= 0 && a < V;
    // a token without a valid target has no gradient (its obar row may be
    // unwritten), whatever g holds
    const float gi = valid ? g[i] : 0.f;
    const bool ok = valid && gi != 0.f;
    const float ct = ok ? -expm1f(logp[i]) : 0.f;
    const uint16_t* wr = w + (int64_t)(ok ? a : 0) * w_ld;
    const float* orow = obar + i * obar_ld;
    uint16_t* out = dh + i * dh_ld;
    for (int d = threadIdx.x * 2; d < H; d += 512) {
      const float w0 = ok ? widen<Tag>(wr[d]) : 0.f, w1 = ok ? widen<Tag>(wr[d + 1]) : 0.f;
      const float v0 = gi == 0.f ? 0.f : gi * (ct * w0 - orow[d]);
      const float v1 = gi == 0.f ? 0.f : gi * (ct * w1 - orow[d + 1]);
      *reinterpret_cast<uint32_t*>(out + d) = pack2<Tag>(v0, v1);
    }
  }
}

int cu_count(int* out) {
  static std::mutex mu;
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    *out = 256;
    return RRL_OK;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  *out = cached[dev];
  return RRL_OK;
}

template <class Tag, int MODE>
int launch_tiles(const LmArgs& a, int64_t H, hipStream_t st) {
  const int64_t nblocks = (a.nx + kBM - 1) / kBM;
  unsigned grid = (unsigned)(a.block_order != nullptr ? nblocks + (nblocks + 1) / 2 : nblocks);
  if (MODE == kModeDw && a.dw_split > 1)
    grid = (unsigned)(a.dw_full + (nblocks - a.dw_full) * a.dw_split);
  if (grid == 0) return RRL_OK;
#define RRL_LM_CASE(HV)                                                                        \
  case HV:                                                                                     \
    hipLaunchKernelGGL((lm_tile_kernel<Tag, MODE, HV>), dim3(grid), dim3(kNT), 0, st, a);      \
    return check_launch("lm_tile_kernel");
  switch (H) {
    RRL_LM_CASE(128)
    RRL_LM_CASE(256)
    RRL_LM_CASE(384)
    RRL_LM_CASE(512)
    RRL_LM_CASE(640)
    RRL_LM_CASE(768)
    RRL_LM_CASE(896)
    RRL_LM_CASE(1024)
    default: break;
  }
#undef RRL_LM_CASE
  set_error("lm head: hidden size must be a multiple of 128 and at most 1024");
  return RRL_EINVAL;
}

// bfloat16 only: the softmax weights and gradients go through the MFMA as
// 16-bit values, and float16's 5-bit exponent cannot hold weights of order
// 1/V (6.6e-6 at V = 151936 is below its 6.1e-5 normal minimum).
template <int MODE>
int launch_tiles_dt(int32_t /*dt*/, const LmArgs& a, int64_t H, hipStream_t st) {
  return launch_tiles<TagBF16, MODE>(a, H, st);
}

int launch_lse(const LmArgs& a, int64_t H, hipStream_t st) {
  const unsigned grid = (unsigned)((a.nx + 2 * kBM - 1) / (2 * kBM));
  if (grid == 0) return RRL_OK;
#define RRL_LSE_CASE(HV)                                                                      \
  case HV:                                                                                    \
    hipLaunchKernelGGL((lm_lse_kernel<TagBF16, HV>), dim3(grid), dim3(kNT), 0, st, a);        \
    return check_launch("lm_lse_kernel");
  switch (H) {
    RRL_LSE_CASE(128)
    RRL_LSE_CASE(256)
    RRL_LSE_CASE(384)
    RRL_LSE_CASE(512)
    RRL_LSE_CASE(640)
    RRL_LSE_CASE(768)
    RRL_LSE_CASE(896)
    RRL_LSE_CASE(1024)
    default: break;
  }
#undef RRL_LSE_CASE
  set_error("lm head: hidden size must be a multiple of 128 and at most 1024");
  return RRL_EINVAL;
}

int check_operands(int32_t dt, int64_t N, int64_t H, int64_t V, const void* hidden,
                   int64_t h_ld, const void* weight, int64_t w_ld) {
  RRL_REQUIRE(dt == RRL_BF16, RRL_EDTYPE, "lm head: hidden and weight must be bfloat16");
  RRL_REQUIRE(N >= 0 && V >= 1 && V < ((int64_t)1 << 31) && N < ((int64_t)1 << 31), RRL_EINVAL,
              "lm head: need 0 <= N < 2^31 tokens and 1 <= V < 2^31");
  RRL_REQUIRE(H >= 128 && H <= 1024 && H % 128 == 0, RRL_EINVAL,
              "lm head: hidden size must be a multiple of 128 and at most 1024");
  RRL_REQUIRE(h_ld >= H && w_ld >= H && h_ld % 8 == 0 && w_ld % 8 == 0, RRL_EINVAL,
              "lm head: row strides must be >= H and multiples of 8 elements");
  RRL_REQUIRE(N == 0 || (hidden && (uintptr_t)hidden % 16 == 0), RRL_EALIGN,
              "lm head: hidden must be 16-byte aligned");
  RRL_REQUIRE(weight && (uintptr_t)weight % 16 == 0, RRL_EALIGN,
              "lm head: weight must be 16-byte aligned");
  // One tile's byte range must fit a buffer descriptor.
  RRL_REQUIRE((int64_t)kBN * (h_ld > w_ld ? h_ld : w_ld) * 2 < ((int64_t)1 << 31), RRL_EINVAL,
              "lm head: row stride too large");
  return RRL_OK;
}

}  // namespace
}  // namespace rrl

using namespace rrl;

extern "C" int rrl_lm_head_fwd(const void* hidden, const void* weight, int32_t dtype, int64_t N,
                               int64_t H, int64_t V, int64_t h_ld, int64_t w_ld,
                               const int32_t* targets, const uint8_t* need_obar,
                               const float* mref_in, float* lse_out, float* logp_out, float* obar,
                               int64_t obar_ld, void* workspace, int32_t* status, void* stream) {
  clear_error();
  if (int rc = check_operands(dtype, N, H, V, hidden, h_ld, weight, w_ld)) return rc;
  if (N == 0) return RRL_OK;
  RRL_REQUIRE(targets && lse_out && logp_out && status, RRL_EINVAL,
              "lm head: null pointer argument");
  RRL_REQUIRE(mref_in == nullptr || obar != nullptr, RRL_EINVAL,
              "lm head: mref_in applies to the pass that forms obar");
  RRL_REQUIRE(obar == nullptr || obar_ld >= H, RRL_EINVAL, "lm head: obar row stride < H");
  LmArgs a{};
  a.x = hidden; a.x_ld = h_ld; a.nx = (int32_t)N;
  a.y = weight; a.y_ld = w_ld; a.ny = (int32_t)V;
  a.V = (int32_t)V;
  a.tgt = targets; a.lse_out = lse_out; a.logp_out = logp_out;
  a.obar = obar; a.obar_ld = obar_ld; a.mref_in = mref_in; a.need_obar = need_obar;
  a.status = status;
  hipStream_t st = as_stream(stream);
  if (!obar) {
    a.need_obar = nullptr;
    return launch_lse(a, H, st);
  }
  if (!need_obar) return launch_tiles_dt<kModeFwd>(dtype, a, H, st);
  RRL_REQUIRE(workspace != nullptr && ((uintptr_t)workspace & 15) == 0, RRL_EINVAL,
              "lm head: need_obar requires a 16-byte aligned workspace of "
              "rrl_lm_head_fwd_workspace_bytes(N) bytes");
  // Blocks that need obar (listed first) take the obar pass, those that need
  // log-probs the log-sum-exp pass, in one launch; blocks that need neither
  // get zeros.
  int32_t* order = static_cast<int32_t*>(workspace);
  hipLaunchKernelGGL(lm_block_order_kernel, dim3(1), dim3(1024), 0, st, (int32_t)N, need_obar,
                     order);
  if (int rc = check_launch("lm_block_order_kernel")) return rc;
  a.block_order = order;
  a.block_count = order + (N + kBM - 1) / kBM;
  return launch_tiles_dt<kModeFwd>(dtype, a, H, st);
}

extern "C" size_t rrl_lm_head_fwd_workspace_bytes(int64_t N) {
  if (N <= 0) return 0;
  return (size_t)(((N + kBM - 1) / kBM + 2) * 4 + 255) / 256 * 256;
}

// Workspace of rrl_lm_head_dweight: 16-byte token records, then the tile
// flags, then the active tile list and its count, then the float32 partial
// rows of the blocks split over tile ranges.
namespace {
size_t records_part(int64_t N) { return ((size_t)(N > 0 ? N : 0) * 16 + 255) & ~(size_t)255; }
size_t flags_part(int64_t N) {
  return ((size_t)((N > 0 ? N : 0) + kBN - 1) / kBN + 255) & ~(size_t)255;
}
size_t list_part(int64_t N) {
  const size_t ntiles = (size_t)((N > 0 ? N : 0) + kBN - 1) / kBN;
  return ((ntiles + 64) * 4 + 255) & ~(size_t)255;
}
// The dW grid: whole blocks, then the blocks of a last partial round of
// workgroups (at most half a round) split into `split` tile ranges each.
struct DwGrid {
  int32_t full, split, rest;
};
DwGrid dw_grid(int64_t V) {
  int cus = 256;
  cu_count(&cus);
  const int64_t nvb = (V + kBM - 1) / kBM;
  const int64_t rest = nvb % cus;
  if (rest == 0 || 2 * rest > cus || nvb < cus) return DwGrid{(int32_t)nvb, 1, 0};
  int64_t split = cus / rest;
  if (split > 8) split = 8;
  return DwGrid{(int32_t)(nvb - rest), (int32_t)split, (int32_t)rest};
}
}  // namespace

extern "C" size_t rrl_lm_head_dweight_workspace_bytes(int64_t N, int64_t H, int64_t V) {
  const DwGrid gd = dw_grid(V > 0 ? V : 0);
  const size_t parts =
      gd.split > 1 ? (size_t)gd.rest * gd.split * kBM * (size_t)(H > 0 ? H : 0) * 4 : 0;
  return records_part(N) + flags_part(N) + list_part(N) + parts;
}

extern "C" int rrl_lm_head_dhidden(const void* weight, int32_t dtype, int64_t N, int64_t H,
                                   int64_t V, int64_t w_ld, const int32_t* targets,
                                   const float* logp, const float* g, const float* obar,
                                   int64_t obar_ld, void* dhidden, int64_t dh_ld,
                                   void* stream) {
  clear_error();
  if (int rc = check_operands(dtype, N, H, V, dhidden, dh_ld, weight, w_ld)) return rc;
  if (N == 0) return RRL_OK;
  RRL_REQUIRE(targets && logp && g && obar && dhidden, RRL_EINVAL,
              "lm head: null pointer argument");
  RRL_REQUIRE(obar_ld >= H, RRL_EINVAL, "lm head: obar row stride < H");
  int cus = 256;
  cu_count(&cus);
  const unsigned grid = (unsigned)(N < 16 * cus ? N : 16 * cus);
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(lm_dhidden_kernel<TagBF16>, dim3(grid), dim3(256), 0, st, N, (int32_t)H,
                     (int32_t)V, static_cast<const uint16_t*>(weight), w_ld, targets, logp, g,
                     obar, obar_ld, static_cast<uint16_t*>(dhidden), dh_ld);
  return check_launch("lm_dhidden_kernel");
}

extern "C" int rrl_lm_head_dweight(const void* hidden, const void* weight, int32_t dtype,
                                   int64_t N, int64_t H, int64_t V, int64_t h_ld, int64_t w_ld,
                                   const int32_t* targets, const float* lse, const float* logp,
                                   const float* g, void* workspace, void* dweight,
                                   int32_t dw_dtype, int64_t dw_ld, void* stream) {
  clear_error();
  if (int rc = check_operands(dtype, N, H, V, hidden, h_ld, weight, w_ld)) return rc;
  RRL_REQUIRE(dw_dtype == RRL_F32 || dw_dtype == dtype, RRL_EDTYPE,
              "lm head: dweight must be float32 or the weight dtype");
  RRL_REQUIRE(dweight && dw_ld >= H, RRL_EINVAL, "lm head: dweight pointer or stride");
  RRL_REQUIRE(N == 0 || (targets && lse && logp && g && workspace), RRL_EINVAL,
              "lm head: null pointer argument");
  RRL_REQUIRE((uintptr_t)workspace % 16 == 0, RRL_EALIGN,
              "lm head: workspace must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint8_t* flags = ws + records_part(N);
  int32_t* list = reinterpret_cast<int32_t*>(flags + flags_part(N));
  float* parts = reinterpret_cast<float*>(flags + flags_part(N) + list_part(N));
  const int64_t ntiles = (N + kBN - 1) / kBN;
  int32_t* count = list + ntiles + 32;
  if (N > 0) {
    int cus = 256;
    cu_count(&cus);
    const unsigned rg = (unsigned)((N + 255) / 256 < 16 * cus ? (N + 255) / 256 : 16 * cus);
    hipLaunchKernelGGL(lm_token_records_kernel, dim3(rg), dim3(256), 0, st, N, (int32_t)V,
                       targets, lse, logp, g, reinterpret_cast<float4*>(ws));
    if (int rc = check_launch("lm_token_records_kernel")) return rc;
    const unsigned fg = (unsigned)((ntiles + 255) / 256 < 4 * cus ? (ntiles + 255) / 256 : 4 * cus);
    hipLaunchKernelGGL(lm_tile_flags_kernel, dim3(fg), dim3(256), 0, st, (int32_t)N, g, flags);
    if (int rc = check_launch("lm_tile_flags_kernel")) return rc;
    hipLaunchKernelGGL(lm_tile_list_kernel, dim3(1), dim3(1024), 0, st, (int32_t)N, flags, list,
                       count);
    if (int rc = check_launch("lm_tile_list_kernel")) return rc;
  }
  LmArgs a{};
  if (N > 0) {
    a.tile_list = list;
    a.tile_count = count;
  }
  a.x = weight; a.x_ld = w_ld; a.nx = (int32_t)V;
  a.y = hidden; a.y_ld = h_ld; a.ny = (int32_t)N;
  a.V = (int32_t)V;
  a.trec = reinterpret_cast<const float4*>(ws);
  a.dw = dweight; a.dw_ld = dw_ld; a.dw_f32 = dw_dtype == RRL_F32;
  const DwGrid gd = dw_grid(V);
  a.dw_full = gd.full;
  a.dw_split = gd.split;
  a.dw_part = gd.split > 1 ? parts : nullptr;
  if (int rc = launch_tiles_dt<kModeDw>(dtype, a, H, st)) return rc;
  if (gd.split > 1) {
    const int32_t nrows = gd.rest * kBM;
    hipLaunchKernelGGL(lm_dw_reduce_kernel<TagBF16>, dim3((unsigned)nrows), dim3(256), 0, st,
                       nrows, gd.split, gd.full, (int32_t)H, (int32_t)V, parts, dweight, dw_ld,
                       (int32_t)a.dw_f32);
    return check_launch("lm_dw_reduce_kernel");
  }
  return RRL_OK;
}
