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
  int64_t out_split_stride;  // elements between split partials (GEMM2)
  int n_ntiles;            // output tiles along Nout
  int splits;              // GEMM2 split-K factor (decode path)
  int group_tiles;         // prefill: concurrent tiles per rasterization window (0 = default)
};

enum class Mode { kGemm1Silu, kGemm2 };
enum class WType { kBf16, kFp8, kInt4 };

}  // namespace fmoe
