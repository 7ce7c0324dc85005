// Wave64 and buffer helpers shared by the register-resident row kernels
// (logprob_resident.hip) and the sampler (sampler.hip), gfx950 only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace rrl {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 2^x with the hardware exponential (v_exp_f32).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Buffer resource over `bytes` bytes at `base`.  The last dword selects a
// non-zero 32-bit data format, which enables raw (untyped) accesses; stride 0
// makes num_records a byte count checked against each access's offset, so a
// load past the end returns zeros and a store past it is dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Cache-policy bits of a buffer access on gfx950: bit 1 = non-temporal.  The
// register-resident kernels read every logit once and write every gradient
// once, so both go non-temporal (the loads measured about 1% faster on the
// fused kernel at config 2 than default-policy loads, in five interleaved
// A/B pairs).
constexpr int kAuxLoad = 2;
constexpr int kAuxStoreNT = 2;

// Butterfly steps inside a row of 16 lanes: DPP quad_perm [1,0,3,2] and
// [2,3,0,1] exchange with lanes i^1 and i^2; once quads agree, the half-row
// and row mirrors pair each half with the other (i^4, i^8 for a reduction).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// Workgroup barrier for LDS exchanges.  __syncthreads()'s release fence waits
// for every outstanding vector-memory access (vmcnt(0)), which would drain
// loads still in flight for a later row or tile; an LDS exchange only needs
// this wave's LDS accesses to have landed, so wait on lgkmcnt alone.
// s_waitcnt immediate, gfx9 layout (bits 3:0 vmcnt[3:0], 6:4 expcnt, 11:8
// lgkmcnt, 15:14 vmcnt[5:4]): 0xC07F = vmcnt 63 and expcnt 7 (no wait),
// lgkmcnt 0.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float lane_read(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Wave64 max / sum / min, the same value in every lane: DPP within rows of
// 16, then the four row results through readlane (scalar operands).
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}
__device__ __forceinline__ int wave_min_dpp(int v) {
  v = min(v, dpp_i<kDppXor1>(v));
  v = min(v, dpp_i<kDppXor2>(v));
  v = min(v, dpp_i<kDppHalfMirror>(v));
  v = min(v, dpp_i<kDppMirror>(v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

}  // namespace
}  // namespace rrl
