// Operand layouts for the chunked LM head's library GEMMs: a transposing copy
// of a 2-byte matrix (the [V, H] LM-head weight into [H, V]).
//
// The GEMM library forms d hidden = dL W fastest (on gfx950, config 5's
// blocks) with the weight held as a contiguous [H, V] matrix; a generic
// strided copy of the 311 MB weight takes 2.5 ms, this one moves it at HBM
// rate.  64 x 64 tiles through LDS: 16-byte loads along the source rows,
// 16-byte stores along the destination rows.
#include "rrl_common.hpp"

namespace rrl {
namespace {

constexpr int kTT = 64;             // tile edge (elements)
constexpr int kTPad = 2;            // LDS row padding (elements)
constexpr int kTThreads = 256;

// dst[c * dst_ld + r] = src[r * src_ld + c] for r < R, c < C.
__global__ __launch_bounds__(kTThreads) void transpose16_kernel(const uint16_t* __restrict__ src,
                                                                int64_t src_ld, int64_t R,
                                                                int64_t C,
                                                                uint16_t* __restrict__ dst,
                                                                int64_t dst_ld, int vec) {
  __shared__ uint16_t tile[kTT][kTT + kTPad];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * kTT, c0 = (int64_t)blockIdx.x * kTT;
  // load: thread t covers source row t/8 (+32), columns 8 (t % 8) .. + 7
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rr = t / 8 + 32 * i, cc = (t % 8) * 8;
    const int64_t r = r0 + rr, c = c0 + cc;
    uint16_t e[8];
    if (r < R && vec && c + 8 <= C) {
      const uint4 v = *reinterpret_cast<const uint4*>(src + r * src_ld + c);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        e[2 * k] = (uint16_t)(w[k] & 0xFFFFu);
        e[2 * k + 1] = (uint16_t)(w[k] >> 16);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = (r < R && c + k < C) ? src[r * src_ld + c + k] : 0;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) tile[rr][cc + k] = e[k];
  }
  __syncthreads();
  // store: thread t covers destination row (source column) t/8 (+32),
  // destination columns (source rows) 8 (t % 8) .. + 7
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int oc = t / 8 + 32 * i, orr = (t % 8) * 8;
    const int64_t c = c0 + oc, r = r0 + orr;
    if (c >= C) continue;
    uint16_t e[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) e[k] = tile[orr + k][oc];
    if (vec && r + 8 <= R) {
      uint4 v;
      v.x = (uint32_t)e[0] | ((uint32_t)e[1] << 16);
      v.y = (uint32_t)e[2] | ((uint32_t)e[3] << 16);
      v.z = (uint32_t)e[4] | ((uint32_t)e[5] << 16);
      v.w = (uint32_t)e[6] | ((uint32_t)e[7] << 16);
      *reinterpret_cast<uint4*>(dst + c * dst_ld + r) = v;
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (r + k < R) dst[c * dst_ld + r + k] = e[k];
    }
  }
}

}  // namespace
}  // namespace rrl

using namespace rrl;

extern "C" int rrl_transpose16(const void* src, int64_t rows, int64_t cols, int64_t src_ld,
                               void* dst, int64_t dst_ld, void* stream) {
  clear_error();
  RRL_REQUIRE(rows >= 0 && cols >= 0, RRL_EINVAL, "rrl_transpose16: negative size");
  if (rows == 0 || cols == 0) return RRL_OK;
  RRL_REQUIRE(src != nullptr && dst != nullptr, RRL_EINVAL, "rrl_transpose16: null operand");
  RRL_REQUIRE(src_ld >= cols && dst_ld >= rows, RRL_EINVAL,
              "rrl_transpose16: a row stride is shorter than its row");
  const int64_t tiles_c = (cols + kTT - 1) / kTT, tiles_r = (rows + kTT - 1) / kTT;
  RRL_REQUIRE(tiles_r <= 65535 && tiles_c <= ((int64_t)1 << 31) - 1, RRL_EINVAL,
              "rrl_transpose16: too many row tiles");
  // 16-byte accesses when every row starts 16-byte aligned
  const int vec = ((uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0 && src_ld % 8 == 0 &&
                   dst_ld % 8 == 0)
                      ? 1
                      : 0;
  hipLaunchKernelGGL(transpose16_kernel, dim3((uint32_t)tiles_c, (uint32_t)tiles_r),
                     dim3(kTThreads), 0, as_stream(stream), static_cast<const uint16_t*>(src),
                     src_ld, rows, cols, static_cast<uint16_t*>(dst), dst_ld, vec);
  return check_launch("transpose16_kernel");
}
