// Shared device helpers for the gfx950 fused-MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmoe.h"

namespace fmoe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin
constexpr float kFp8Max = 448.0f;
constexpr float kFp8Eps = 1e-10f;

// ---------------------------------------------------------------- numerics
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round to nearest even (NaN kept quiet), as torch's .to(bfloat16).
// Written as a select, not an early return: the compiler turns the early
// return into a divergent branch per value (~15 exec-mask instructions), which
// made the GEMM epilogues several times longer than their arithmetic.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;
  return static_cast<uint16_t>((u & 0x7fffffffu) > 0x7f800000u ? qnan : rne);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// v / s correctly rounded (as a plain division, s > 0), then clamped to the
// e4m3 range: v * (1/s) plus one FMA-residual correction (inv = 1/s, itself
// correctly rounded), which restores the rounding the reciprocal product alone
// can miss.  Cheaper than a division per element.  The correction step turns
// a -0 quotient into +0 (+0 + -0), so the sign is copied back from q0, which
// has v's sign like the division (-0 / s = -0, the e4m3 byte 0x80); taking
// it from q0 rather than v keeps v's live range (and the kernels' register
// counts) as without the fix.
__device__ __forceinline__ float fp8_qdiv(float v, float s, float inv) {
  const float q0 = v * inv;
  const float r = __builtin_fmaf(-q0, s, v);
  const float q = __builtin_copysignf(__builtin_fmaf(r, inv, q0), q0);
  return fminf(fmaxf(q, -kFp8Max), kFp8Max);
}

// Four values in the e4m3 range -> packed OCP e4m3 bytes (hardware RNE
// conversion; byte i = value i).
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
  const int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true));
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  // ops/fused_moe.py:46 — gate / (1 + exp(-gate)) * up, in fp32
  return (g / (1.0f + __expf(-g))) * u;
}

// ------------------------------------------------------------- wave utils
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// XCD-aware remap of a linear workgroup id over `count` live workgroups:
// hardware hands consecutive ids to different XCDs; this makes each XCD's
// share a contiguous range of logical tiles so neighbouring tiles (same
// expert, same weight panel) meet in one XCD's L2.
__device__ __forceinline__ int xcd_remap(int b, int count) {
  int x = b % kNumXcd, i = b / kNumXcd;
  int q = count / kNumXcd, r = count % kNumXcd;
  return x * q + (x < r ? x : r) + i;
}

}  // namespace fmoe

// Host-side error reporting shared by the entry points.
namespace fmoe_host {
int fail(int status, const char* fmt, ...);
int check_launch(const char* what);
}  // namespace fmoe_host
