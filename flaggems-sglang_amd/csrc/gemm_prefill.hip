// Prefill grouped GEMM: LDS-staged MFMA tiles, one expert per M-tile.
//
// Workgroup = 256 threads (4 waves, 2 x 2), tile BM x BN, 128 bytes of the
// reduction dim per pipeline stage (bf16: 64 elements, fp8: 128 = one scale
// block), double-buffered in LDS with one barrier per stage.  Each wave owns a
// (BM/2) x (BN/2) sub-tile computed with 16x16 MFMA blocks:
//   bf16: v_mfma_f32_16x16x32_bf16, two per stage;
//   fp8 : v_mfma_f32_16x16x128_f8f6f4 (OCP e4m3), one per stage, its result
//         scaled by a_scale[row] * w_scale[block] into the fp32 accumulator.
// Both operands are read from LDS as 32 contiguous bytes per lane (lane group
// g = lane/16 takes bytes 32g..32g+31 of the stage); A and B use the same
// lane -> k assignment, so the dot products are exact permutations of the
// textbook ones.  LDS rows are padded to 144 bytes: the 16 rows read by one
// quarter-wave then start on distinct 4-bank groups.
//
// GEMM1 (gate/up + SiLU): the BN weight rows of a tile are BN/2 gate rows
// and the matching BN/2 up rows, arranged so every wave holds gate block j
// and up block j in the same lanes; silu(gate) * up is formed in registers
// and only the bf16 activation is written (no intermediate in HBM).
// GEMM2: rows scaled by the routing weight, fp32 partial written per slot;
// the top-k sum runs in fmoe_moe_sum in fixed order.
#include "gemm.hpp"

namespace fmoe {
namespace prefill {

constexpr int kThreads = 256;
constexpr int kStageBytes = 128;  // reduction bytes per stage and row
constexpr int kRowBytes = kStageBytes + 16;
constexpr int kGroupM = 8;        // M-tiles per swizzle group

template <int BM, int BN, bool FP8, Mode MODE>
struct Tile {
  static constexpr int WM = BM / 2, WN = BN / 2;
  static constexpr int MI = WM / 16, NI = WN / 16;
  static constexpr int A_CHUNKS = BM * (kStageBytes / 16) / kThreads;
  static constexpr int B_CHUNKS = BN * (kStageBytes / 16) / kThreads;
  static constexpr int LDS_STAGE = (BM + BN) * kRowBytes;
  static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small");
  static_assert(MODE != Mode::kGemm1Silu || NI % 2 == 0, "gate/up pairing needs even NI");
};

__device__ __forceinline__ void mfma_step(f32x4_t& c, const i32x8_t& a, const i32x8_t& b,
                                          bool fp8) {
  if (fp8) {
    c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  } else {
    bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, i32x4_t{a[0], a[1], a[2], a[3]});
    bf16x8_t b0 = __builtin_bit_cast(bf16x8_t, i32x4_t{b[0], b[1], b[2], b[3]});
    bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, i32x4_t{a[4], a[5], a[6], a[7]});
    bf16x8_t b1 = __builtin_bit_cast(bf16x8_t, i32x4_t{b[4], b[5], b[6], b[7]});
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, c, 0, 0, 0);
  }
}

__device__ __forceinline__ i32x8_t lds_frag(const uint8_t* base) {
  i32x4_t lo = *reinterpret_cast<const i32x4_t*>(base);
  i32x4_t hi = *reinterpret_cast<const i32x4_t*>(base + 16);
  return i32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <int BM, int BN, bool FP8, Mode MODE>
__global__ __launch_bounds__(kThreads) void gemm_prefill_kernel(GemmParams p) {
  using T = Tile<BM, BN, FP8, MODE>;
  constexpr int WM = T::WM, WN = T::WN, MI = T::MI, NI = T::NI;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * T::LDS_STAGE];
  __shared__ float sa_lds[FP8 ? 2 : 1][FP8 ? BM : 1];

  const int tid = threadIdx.x, lane = tid % kWave, wid = tid / kWave;
  const int wm = wid / 2, wn = wid % 2;

  // ---- which (M-tile, N-tile): XCD-contiguous, then grouped along M
  const int n_tiles = *p.n_tiles;
  const int live = n_tiles * p.n_ntiles;
  if (static_cast<int>(blockIdx.x) >= live) return;
  const int L = xcd_remap(blockIdx.x, live);
  const int per_group = kGroupM * p.n_ntiles;
  const int first_m = (L / per_group) * kGroupM;
  const int gsize = min(n_tiles - first_m, kGroupM);
  const int mt = first_m + (L % per_group) % gsize;
  const int nt = (L % per_group) / gsize;

  const int tm = p.tile_map[mt];
  const int e = tm & 0xffff, blk = tm >> 16;
  const int row_beg = p.offs_raw[e] + blk * BM;
  const int row_end = min(p.offs_raw[e + 1], row_beg + BM);

  const int64_t kbytes = FP8 ? p.Kred : p.Kred * 2;  // bytes per operand row
  const int nk = static_cast<int>(kbytes / kStageBytes);
  const int ksb = static_cast<int>(p.Kred / 128);      // fp8 scale blocks per row

  // ---- per-thread global source rows
  const int c16 = tid & 7;
  const uint8_t* a_src[T::A_CHUNKS];
#pragma unroll
  for (int i = 0; i < T::A_CHUNKS; ++i) {
    int r = (tid >> 3) + i * (kThreads / 8);
    int s = row_beg + r;
    if (s >= row_end) s = row_beg;  // padding row: any valid row, result discarded
    int64_t src = MODE == Mode::kGemm1Silu ? p.topk_indx[s] / p.top_k : s;
    a_src[i] = p.A + src * kbytes + c16 * 16;
  }
  const uint8_t* b_src[T::B_CHUNKS];
  const uint8_t* Be = p.B + static_cast<int64_t>(e) * p.Nout * kbytes;
#pragma unroll
  for (int i = 0; i < T::B_CHUNKS; ++i) {
    int r = (tid >> 3) + i * (kThreads / 8);
    int64_t brow;
    if (MODE == Mode::kGemm1Silu) {
      int w = r / WN, within = r % WN;
      int64_t j = static_cast<int64_t>(nt) * (BN / 2) + w * (WN / 2) + (within % (WN / 2));
      brow = within < WN / 2 ? j : p.N_act + j;
    } else {
      brow = static_cast<int64_t>(nt) * BN + r;
      if (brow >= p.Nout) brow = p.Nout - 1;
    }
    b_src[i] = Be + brow * kbytes + c16 * 16;
  }
  const float* sa_src = nullptr;
  if (FP8 && tid < BM) {
    int s = row_beg + tid;
    if (s >= row_end) s = row_beg;
    int64_t src = MODE == Mode::kGemm1Silu ? p.topk_indx[s] / p.top_k : s;
    sa_src = p.a_scale + src * ksb;
  }
  // fp8 weight-scale rows for this wave (gate / up blocks, or the GEMM2 block)
  const float* sb_src0 = nullptr;
  const float* sb_src1 = nullptr;
  if (FP8) {
    const int64_t nrb = p.Nout / 128;
    const float* se = p.b_scale + static_cast<int64_t>(e) * nrb * ksb;
    if (MODE == Mode::kGemm1Silu) {
      int64_t j = static_cast<int64_t>(nt) * (BN / 2) + wn * (WN / 2);
      sb_src0 = se + (j / 128) * ksb;
      sb_src1 = se + ((p.N_act + j) / 128) * ksb;
    } else {
      int64_t j = static_cast<int64_t>(nt) * BN + wn * WN;
      if (j >= p.Nout) j = p.Nout - 1;
      sb_src0 = se + (j / 128) * ksb;
      sb_src1 = sb_src0;
    }
  }

  i32x4_t ra[T::A_CHUNKS], rb[T::B_CHUNKS];
  float rsa = 0.f;
  auto gload = [&](int kt) {
    const int64_t off = static_cast<int64_t>(kt) * kStageBytes;
#pragma unroll
    for (int i = 0; i < T::A_CHUNKS; ++i) ra[i] = *reinterpret_cast<const i32x4_t*>(a_src[i] + off);
#pragma unroll
    for (int i = 0; i < T::B_CHUNKS; ++i) rb[i] = *reinterpret_cast<const i32x4_t*>(b_src[i] + off);
    if (FP8 && sa_src) rsa = sa_src[kt];
  };
  auto lstore = [&](int buf) {
    uint8_t* As = lds + buf * T::LDS_STAGE;
    uint8_t* Bs = As + BM * kRowBytes;
#pragma unroll
    for (int i = 0; i < T::A_CHUNKS; ++i) {
      int r = (tid >> 3) + i * (kThreads / 8);
      *reinterpret_cast<i32x4_t*>(As + r * kRowBytes + c16 * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < T::B_CHUNKS; ++i) {
      int r = (tid >> 3) + i * (kThreads / 8);
      *reinterpret_cast<i32x4_t*>(Bs + r * kRowBytes + c16 * 16) = rb[i];
    }
    if (FP8 && tid < BM) sa_lds[buf][tid] = rsa;
  };

  f32x4_t acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  gload(0);
  lstore(0);
  __syncthreads();

  const int frag_off = (lane & 15) * kRowBytes + (lane >> 4) * 32;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const uint8_t* As = lds + cur * T::LDS_STAGE;
    const uint8_t* Bs = As + BM * kRowBytes;
    i32x8_t fa[MI], fb[NI];
#pragma unroll
    for (int i = 0; i < MI; ++i) fa[i] = lds_frag(As + (wm * WM + i * 16) * kRowBytes + frag_off);
#pragma unroll
    for (int j = 0; j < NI; ++j) fb[j] = lds_frag(Bs + (wn * WN + j * 16) * kRowBytes + frag_off);
    if (FP8) {
      const float sb0 = sb_src0[kt], sb1 = sb_src1[kt];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        float sa[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sa[r] = sa_lds[cur][wm * WM + i * 16 + (lane >> 4) * 4 + r];
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          f32x4_t t = {0.f, 0.f, 0.f, 0.f};
          mfma_step(t, fa[i], fb[j], true);
          const float sb = (MODE == Mode::kGemm1Silu && j >= NI / 2) ? sb1 : sb0;
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] += t[r] * (sa[r] * sb);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) mfma_step(acc[i][j], fa[i], fb[j], false);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue.  C layout of a 16x16 block: lane holds column lane%16,
  // rows 4*(lane/16) + r.
  const int col16 = lane & 15;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int s = row_beg + wm * WM + i * 16 + (lane >> 4) * 4 + r;
      if (s >= row_end) continue;
      const float g = p.gamma ? p.gate_scal[s] : 1.0f;
      if (MODE == Mode::kGemm1Silu) {
        uint16_t* act = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(s) * p.N_act;
#pragma unroll
        for (int j = 0; j < NI / 2; ++j) {
          const float gv = round_bf16(acc[i][j][r] * g);
          const float uv = round_bf16(acc[i][j + NI / 2][r] * g);
          const int64_t col = static_cast<int64_t>(nt) * (BN / 2) + wn * (WN / 2) + j * 16 + col16;
          act[col] = f32_to_bf16(silu_mul(gv, uv));
        }
      } else {
        float* y = static_cast<float*>(p.out) + static_cast<int64_t>(s) * p.Nout;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int64_t col = static_cast<int64_t>(nt) * BN + wn * WN + j * 16 + col16;
          if (col < p.Nout) y[col] = acc[i][j][r] * g;
        }
      }
    }
  }
}

}  // namespace prefill

// Host launcher: picks the instantiation.
int launch_prefill(WType wt, Mode mode, int bm, const GemmParams& p0, hipStream_t s) {
  GemmParams p = p0;
  constexpr int BN = 256;
  const int64_t ncols = mode == Mode::kGemm1Silu ? p.N_act : p.Nout;
  const int per_tile = mode == Mode::kGemm1Silu ? BN / 2 : BN;
  p.n_ntiles = static_cast<int>((ncols + per_tile - 1) / per_tile);
  const int64_t grid = static_cast<int64_t>(p.max_tiles) * p.n_ntiles;
  if (grid <= 0) return FMOE_OK;
  if (grid > 0x7fffffff) return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "prefill grid too large");
  dim3 g(static_cast<unsigned>(grid)), b(prefill::kThreads);
#define LAUNCH(BM_, FP8_, MODE_) \
  prefill::gemm_prefill_kernel<BM_, BN, FP8_, MODE_><<<g, b, 0, s>>>(p)
  const bool fp8 = wt == WType::kFp8;
  if (bm == 128) {
    if (mode == Mode::kGemm1Silu) {
      if (fp8) LAUNCH(128, true, Mode::kGemm1Silu); else LAUNCH(128, false, Mode::kGemm1Silu);
    } else {
      if (fp8) LAUNCH(128, true, Mode::kGemm2); else LAUNCH(128, false, Mode::kGemm2);
    }
  } else if (bm == 64) {
    if (mode == Mode::kGemm1Silu) {
      if (fp8) LAUNCH(64, true, Mode::kGemm1Silu); else LAUNCH(64, false, Mode::kGemm1Silu);
    } else {
      if (fp8) LAUNCH(64, true, Mode::kGemm2); else LAUNCH(64, false, Mode::kGemm2);
    }
  } else {
    return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "prefill: block_m=%d is not supported", bm);
  }
#undef LAUNCH
  return fmoe_host::check_launch("gemm_prefill");
}

}  // namespace fmoe
