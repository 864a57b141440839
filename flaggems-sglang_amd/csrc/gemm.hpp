// Shared definitions of the grouped (per-expert) MoE GEMM kernels.
#pragma once

#include "common.hpp"

namespace fmoe {

// One launch = one of the two expert GEMMs over every (expert tile, output
// tile) pair.  Operand "A" is the activation side (rows = slots), "B" the
// expert weights stored [E, Nout, Kred] (reduction dim contiguous, the SGLang
// layer layout), so both MFMA operands read contiguous K from memory.
struct GemmParams {
  const uint8_t* A;        // GEMM1: x [M, Kred]; GEMM2: act [M*k, Kred]
  const float* a_scale;    // fp8: [rows, Kred/128]
  const uint8_t* B;        // [E, Nout, Kred] elements (int4: packed, Kred/2 bytes per row)
  const float* b_scale;    // fp8: [E, Nout/128, Kred/128]
  const uint16_t* b_gscale;  // int4: fp16 [E, Kred/128, Nout]
  const uint8_t* b_zero;   // int4: u4 [E, Kred/128, Nout/2]
  const uint8_t* b_mxscale;  // mxfp4: e8m0 [E, Nout, Kred/32]
  int b_tiled;             // int4: B in the 16-row x 128-element tiled layout
                           // (FMOE_W_INT4_TILED) instead of row-major
  int64_t Kred;            // reduction length (elements)
  int64_t Nout;            // weight rows per expert (GEMM1: 2N, GEMM2: K)
  int64_t N_act;           // GEMM1: N (columns of act)
  const int32_t* topk_indx;
  const float* gate_scal;
  const int32_t* offs_raw;
  const int32_t* offs_pad;   // [E+1] tile offsets per expert
  const int32_t* tile_map;
  const int32_t* n_tiles;
  int top_k;
  int n_experts;
  int max_tiles;
  int gamma;               // multiply rows by gate_scal[slot]
  void* out;               // GEMM1: act bf16 [M*k, N]; GEMM2: y fp32 [splits][M*k, Nout]
  int y_bf16;              // prefill GEMM2 with one split: y rows stored as bf16 instead
  // fp8 prefill GEMM1: when set, the activation leaves the epilogue already
  // quantized (e4m3 [M*k, N] + fp32 scales [M*k, N/128]) instead of as bf16
  uint8_t* act_q;
  float* act_qs;
  int64_t out_split_stride;  // elements between split partials (GEMM2)
  int n_ntiles;            // output tiles along Nout
  int splits;              // GEMM2 split-K factor (decode path)
  int group_tiles;         // prefill: concurrent tiles per rasterization window (0 = default)
  // prefill: optional [n_tiles * n_ntiles] table, logical tile ->
  // (expert, N-tile, first row, end row), filled by a small kernel before the
  // GEMM (replaces the dependent routing loads of every workgroup's prologue)
  int4* tile_lut;
  // prefill GEMM2 tail split (0 = off): each XCD's logical tiles run whole
  // (bf16 rows, y_bf16) except the last partial round's, which are split up
  // to tail_split ways along the reduction dim so they fill one round of the
  // XCD's tail_slots workgroup slots; their fp32 partials go to tail_part
  // ([pair][BM][BN], pairs numbered XCD by XCD, tile * S + split within one) and
  // tail_fold_kernel adds them into the bf16 rows
  int tail_split;
  int tail_slots;
  float* tail_part;
  int64_t tail_pairs;  // capacity of tail_part in [BM][BN] partials (set by the launcher)
  size_t tail_bytes;   // size of tail_part
  // epilogue (fmoe_epilogue): activation, fp32 bias [E, Nout], swiglu alpha / limit
  int act;
  const float* bias;
  float alpha;
  float limit;
  // tiny-batch decode path (routing computed in each workgroup, no align
  // launch): topk ids / weights [n_tokens * top_k]; rows are flat slots
  const int32_t* tiny_ids;
  const float* tiny_w;
  int64_t n_tokens;
};

enum Act { kActSilu = 0, kActGelu = 1, kActSwiglu = 2 };

enum class Mode { kGemm1Silu, kGemm2 };
enum class WType { kBf16, kFp8, kInt4, kMxfp4 };
constexpr int kTailMaxSplit = 4;  // prefill GEMM2 tail split: ways per tail tile

// Weight row of GEMM1 output column c: gate (u = 0) or up / linear (u = 1).
// SiLU and GELU use split halves (gate c, up N + c), SWIGLU interleaved rows
// (gate 2c, linear 2c + 1).
__host__ __device__ __forceinline__ int64_t gemm1_row(int act, int64_t n_act, int64_t c, int u) {
  return act == kActSwiglu ? 2 * c + u : c + u * n_act;
}

// GEMM1 epilogue value for output column c of a slot (ACT = the
// activation, a template parameter so each kernel variant carries only its
// own epilogue): ga / ua are the fp32 GEMM results of its gate and up
// (linear) rows, gb / ub their biases, g the routing weight when applied on
// the input (else 1).
template <int ACT>
__device__ __forceinline__ float gemm1_act(const GemmParams& p, float ga, float ua, float gb,
                                           float ub, float g) {
  if constexpr (ACT == kActSwiglu) {
    float gv = ga + gb, lv = ua + ub;
    if (p.limit > 0.f) {
      gv = fminf(gv, p.limit);
      lv = fminf(fmaxf(lv, -p.limit), p.limit);
    }
    return gv / (1.0f + __expf(-p.alpha * gv)) * (lv + 1.0f) * g;
  } else {
    const float gv = round_bf16(ga * g), uv = round_bf16(ua * g);
    if constexpr (ACT == kActGelu) return 0.5f * gv * (1.0f + erff(gv * 0.7071067811865476f)) * uv;
    return silu_mul(gv, uv);
  }
}

// GEMM1 biases of output column c of expert e (0 without a bias; only the
// SWIGLU variant takes one).
template <int ACT>
__device__ __forceinline__ void gemm1_bias(const GemmParams& p, int e, int64_t c, float& gb,
                                           float& ub) {
  gb = ub = 0.f;
  if constexpr (ACT == kActSwiglu) {
    if (p.bias) {
      const float* b = p.bias + static_cast<int64_t>(e) * p.Nout;
      gb = b[gemm1_row(ACT, p.N_act, c, 0)];
      ub = b[gemm1_row(ACT, p.N_act, c, 1)];
    }
  }
}

}  // namespace fmoe
