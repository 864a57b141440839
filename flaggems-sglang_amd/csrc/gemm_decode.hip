// Decode grouped GEMM: weights streamed straight from HBM into MFMA registers.
//
// For small token counts every expert tile holds <= 16 slots, so the work is
// bound by reading each touched expert's weights once.  A workgroup (4
// waves) owns 16 slots x 64 weight rows and splits the reduction dim between
// its waves by interleaved stages (wave w takes stages w, w+4, ...), so at any
// moment the four waves read adjacent pieces of the same 64 rows; lane group
// g = lane/16 reads its part of row lane%16 of each 16-row block.  The fp8
// GEMM1 variant with in-workgroup routing (tiny batches) and the MXFP4
// variants keep two stages of loads in flight per wave (their in-register
// activation quantization / e2m1 conversion is long enough to hide a second
// stage behind); every other variant issues one stage at a time, which keeps
// VGPR use and therefore occupancy higher -- measured faster (see
// pipe_depth).  No LDS staging;
// the per-wave partial accumulators are summed through LDS once at the end.
// GEMM2 may further split the reduction across workgroups (`splits`); the
// partials land in separate y planes that fmoe_moe_sum adds in fixed order.
// A workgroup may hold RB such row blocks (RB x 4 waves, RB x 64 rows; the
// waves of one reduction slice then read the same activation bytes): chosen
// per format by measurement (decode_row_blocks).
//
// 4-bit weights (int4, MXFP4) come row-major ([rows][K/2]: one load
// instruction touches 16 rows x 64 bytes, half cache lines) or tiled
// (FMOE_W_INT4_TILED / FMOE_W_MXFP4_TILED: each 16-row x 64-byte block stored
// contiguously in lane order, so the same instruction reads one contiguous
// KiB); only the addresses differ, results are identical.
//
// Weight formats (one stage = one 128-byte slice of a weight row, int4: 64):
//   bf16: 16 elements per lane -> two v_mfma_f32_16x16x32_bf16.
//   fp8 : 32 elements per lane -> one v_mfma_f32_16x16x128_f8f6f4, scaled by
//         a_scale * w_scale per 128-wide block.  The activation side arrives as
//         bf16 and is quantized here, per row and 128-group, to OCP e4m3 with
//         scale = max(amax, 1e-10) / 448 (amax reduced over the 4 lane groups
//         holding the row, hardware RNE conversion) -- no separate quant pass.
//   int4: 32 nibbles per lane (one 128-wide quant group per stage).  A nibble
//         q becomes the bf16 number 128 + q by OR-ing 0x4300 into its 16-bit
//         lane (exact: bf16 spacing at 128 is 1), so the MFMA computes
//         sum((128 + q) x); with xs = sum(x) over the group (an MFMA against a
//         ones vector) the dequantized product is
//         scale * (sum((128+q) x) - (128 + zero) * xs).
//         The nibble pairs come out as k = (j, j+4) of each 8-nibble dword;
//         the activations are permuted the same way with v_perm_b32.

#include <type_traits>

#include "gemm.hpp"

namespace fmoe {
namespace decode {

constexpr int kThreads = 256;  // one row block: 4 waves
constexpr int kWaves = 4;      // waves splitting the reduction dim of a row block
constexpr int kMaxRB = 2;
constexpr int BM = 16;
constexpr int BN = 64;
constexpr int NI = BN / 16;

__device__ __forceinline__ i32x8_t gload32(const uint8_t* p) {
  i32x4_t lo = *reinterpret_cast<const i32x4_t*>(p);
  i32x4_t hi = *reinterpret_cast<const i32x4_t*>(p + 16);
  return i32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ bf16x8_t as_bf16x8(int a, int b, int c, int d) {
  return __builtin_bit_cast(bf16x8_t, i32x4_t{a, b, c, d});
}

// Per-stage operand registers of one wave.
template <WType WT>
struct Stage;
template <>
struct Stage<WType::kBf16> {
  i32x8_t a;      // 16 bf16 of the activation row
  i32x8_t b[NI];  // 16 bf16 of each weight row
};
template <>
struct Stage<WType::kFp8> {
  i32x4_t a[4];   // 32 bf16 of the activation row (quantized in registers)
  i32x8_t b[NI];  // 32 fp8 of each weight row
  float sb[NI];   // weight block scale of each 16-row block
};
template <>
struct Stage<WType::kInt4> {
  i32x4_t a[4];   // 32 bf16 of the activation row
  i32x4_t b[NI];  // 32 uint4 of each weight row
  int meta;       // one dword of the wave's group scales / zeros (see int4_meta)
};

template <>
struct Stage<WType::kMxfp4> {
  i32x4_t a[4];     // 32 bf16 of the activation row
  i32x4_t b[NI];    // 32 e2m1 of each weight row (one 32-element scale block)
  uint8_t sx[NI];   // e8m0 scale of that block
};

// Stages in flight per wave (see the file comment).
// (fp8 GEMM1 with in-workgroup routing: two, measured faster at M = 1; with
// the align launch, e.g. DSV3 M = 128, one stage and twice the occupancy is
// 7% faster.  MXFP4: two, 3-5% faster at M = 16 (its e2m1 conversions hide
// the second stage), even at M = 1.  bf16 / int4: one.)
constexpr int pipe_depth(WType wt, Mode mode, bool tiny) {
  if (wt == WType::kInt4) return 1;
  return (wt == WType::kFp8 && mode == Mode::kGemm1Silu && tiny) || wt == WType::kMxfp4 ? 2 : 1;
}

// Issue priority of a wave while it consumes a stage (its loads are out):
// raised for bf16 (Mixtral M=16 480 -> 461 us, Qwen3 M=64 217 -> 210 us);
// fp8 (DSV3 M=1 +5%) and int4 (neutral) keep one level.
template <WType WT>
constexpr int decode_prio() { return WT == WType::kBf16 ? 1 : 0; }

// Tiny batches (tiles of <= 16 slots, at most kTinySlots slots): the routing
// of one tile computed inside the workgroup from the top-k ids, replacing
// the align launch.  Tiles are the (expert, 16-slot block) pairs of the
// experts in ascending order, slots of an expert in ascending flat order
// t * k + j -- the same tiles, in the same order, as the align kernels
// produce, so results are identical; a tile's rows are flat slot indices.
constexpr int kTinySlots = 512;
constexpr int kTinyExperts = 1024;

struct TinyLds {
  int cnt[kTinyExperts];
  int ids[kTinySlots];
  int rows[BM];
  int info[4];     // expert, block, rows in the tile, valid
  int scan[16];    // one entry per wave (up to 16 waves)
};

// Returns false when tile mt does not exist (same decision in every thread).
// NT = threads of the workgroup.
template <int NT>
__device__ bool tiny_route(const GemmParams& p, int mt, TinyLds& L) {
  static_assert(NT % kWave == 0 && NT / kWave <= 16, "tiny_route: up to 16 waves");
  const int tid = threadIdx.x, lane = tid % kWave, wid = tid / kWave;
  const int E = p.n_experts;
  const int n = static_cast<int>(p.n_tokens * p.top_k);
  for (int e = tid; e < E; e += NT) L.cnt[e] = 0;
  if (tid == 0) L.info[3] = 0;
  __syncthreads();
  for (int f = tid; f < n; f += NT) {
    const int id = p.tiny_ids[f];
    L.ids[f] = id;
    if (id >= 0 && id < E) atomicAdd(&L.cnt[id], 1);
  }
  __syncthreads();
  // tiles per expert = ceil(count / 16); thread t owns experts [t*per, t*per+per)
  const int per = (E + NT - 1) / NT;
  int mine = 0;
  for (int i = 0; i < per; ++i) {
    const int e = tid * per + i;
    if (e < E) mine += (L.cnt[e] + BM - 1) / BM;
  }
  int x = mine;  // inclusive scan over the workgroup
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == kWave - 1) L.scan[wid] = x;
  __syncthreads();
  int base = x - mine;
  for (int w = 0; w < wid; ++w) base += L.scan[w];
  if (mt >= base && mt < base + mine) {
    int t = base;
    for (int i = 0; i < per; ++i) {
      const int e = tid * per + i;
      const int nt = e < E ? (L.cnt[e] + BM - 1) / BM : 0;
      if (mt < t + nt) {
        const int blk = mt - t;
        L.info[0] = e;
        L.info[1] = blk;
        L.info[2] = min(BM, L.cnt[e] - blk * BM);
        L.info[3] = 1;
        break;
      }
      t += nt;
    }
  }
  __syncthreads();
  if (!L.info[3]) return false;
  // rows: the [blk*16, blk*16+16) occurrences of expert e in flat order
  const int e = L.info[0], lo = L.info[1] * BM;
  int run = 0;
  for (int c0 = 0; c0 < n; c0 += NT) {
    const int f = c0 + tid;
    const bool hit = f < n && L.ids[f] == e;
    const uint64_t m = __ballot(hit);
    const int before = __popcll(m & ((1ull << lane) - 1ull));
    __syncthreads();  // L.scan reuse
    if (lane == 0) L.scan[wid] = __popcll(m);
    __syncthreads();
    int off = run;
    for (int w = 0; w < wid; ++w) off += L.scan[w];
    const int pos = off + before;
    if (hit && pos >= lo && pos < lo + BM) L.rows[pos - lo] = f;
    for (int w = 0; w < NT / kWave; ++w) run += L.scan[w];
  }
  __syncthreads();
  return true;
}

template <WType WT, Mode MODE, int PIPE, int ACT, bool TINY, int RB>
__global__ __launch_bounds__(kThreads * RB, WT == WType::kInt4 ? 4 : 1) void gemm_decode_kernel(GemmParams p) {
  __shared__ f32x4_t red[RB][kWaves][NI][kWave];
  __shared__ TinyLds tiny_lds[1];  // used by the TINY variant only
  const int tid = threadIdx.x, lane = tid % kWave;
  // wave index as a scalar: the compiler then treats the per-wave stage
  // schedule (kw, k ranges, "more" stages) as uniform, so its loads sit under
  // scalar branches and the waits before their uses count exactly
  const int wid = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int kw = wid % kWaves;  // reduction-dim slice of this wave
  const int rb = wid / kWaves;  // row block of this wave
  int mt = blockIdx.x, ntw = blockIdx.y, split = blockIdx.z;
  if constexpr (!TINY) {
    // Only the first n_tiles x gridDim.y x gridDim.z workgroups have work;
    // their ids are remapped so each XCD takes a contiguous run of the
    // logical order, in which neighbours share data that then meets in one
    // XCD's L2 instead of being fetched by every XCD:
    //  * short tiles (<= 128 row workgroups: DSV3, Qwen3 shapes): row blocks
    //    fastest, so a tile's activation rows are read by one or two XCDs;
    //  * long tiles (Mixtral): tiles fastest, so the tiles of one expert at
    //    the same row block (the same weight bytes) run side by side.
    const int gy = gridDim.y;
    const int ntl = *p.n_tiles;
    const int live = ntl * gy * gridDim.z;
    const int b = blockIdx.x + gridDim.x * (blockIdx.y + gy * blockIdx.z);
    if (b >= live) return;
    const int L = xcd_remap(b, live);
    split = L / (gy * ntl);
    if (gy <= 128) {
      ntw = L % gy;
      mt = (L / gy) % ntl;
    } else {
      mt = L % ntl;
      ntw = (L / ntl) % gy;
    }
  }
  const int nt = ntw * RB + rb;  // 64-row block index

  // this tile: expert e and its rows (slot of tile row r = slot_of(r), r < n_rows)
  int e, row_beg = 0, n_rows;
  if constexpr (TINY) {
    if (!tiny_route<kThreads * RB>(p, mt, tiny_lds[0])) return;
    e = tiny_lds[0].info[0];
    n_rows = tiny_lds[0].info[2];
  } else {
    if (mt >= *p.n_tiles) return;  // tile slot beyond this call's tiles
    const int tm = p.tile_map[mt];
    e = tm & 0xffff;
    const int blk = tm >> 16;
    row_beg = p.offs_raw[e] + blk * BM;
    n_rows = min(p.offs_raw[e + 1], row_beg + BM) - row_beg;
  }
  auto slot_of = [&](int r) { return TINY ? tiny_lds[0].rows[r] : row_beg + r; };

  constexpr bool kFp8 = WT == WType::kFp8;
  constexpr bool kInt4 = WT == WType::kInt4;
  constexpr bool kMx = WT == WType::kMxfp4;
  constexpr bool kNib = kInt4 || kMx;  // 4-bit weights, two per byte
  // A rows: row lane%16 of the tile (bf16 for every format)
  const int s_a = slot_of((lane & 15) < n_rows ? (lane & 15) : 0);
  const int64_t a_row = MODE == Mode::kGemm1Silu ? (TINY ? s_a : p.topk_indx[s_a]) / p.top_k : s_a;
  const uint8_t* a_ptr = p.A + a_row * p.Kred * 2;
  // stage geometry
  constexpr int kWStage = kNib ? 64 : 128;          // weight bytes per row per stage
  constexpr int kElems = kNib ? 128 : (kFp8 ? 128 : 64);  // reduction elements per stage
  const int64_t w_bytes = kNib ? p.Kred / 2 : (kFp8 ? p.Kred : p.Kred * 2);
  const int nk = static_cast<int>(w_bytes / kWStage);
  const int lane_off_w = (lane >> 4) * (kNib ? 16 : 32);
  const int lane_off_a = (lane >> 4) * (WT == WType::kBf16 ? 32 : 64);  // bf16 activations

  const uint8_t* Be = p.B + static_cast<int64_t>(e) * p.Nout * w_bytes;
  int64_t wrow[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    int64_t r;
    if (MODE == Mode::kGemm1Silu) {
      int64_t jj = static_cast<int64_t>(nt) * (BN / 2) + (j % (NI / 2)) * 16 + (lane & 15);
      if (jj >= p.N_act) jj = p.N_act - 1;  // last row block of an RB > 1 grid
      r = gemm1_row(ACT, p.N_act, jj, j < NI / 2 ? 0 : 1);
    } else {
      r = static_cast<int64_t>(nt) * BN + j * 16 + (lane & 15);
      if (r >= p.Nout) r = p.Nout - 1;
    }
    wrow[j] = r;
  }
  // Weight row r's stage-kt slice: row-major at r * w_bytes + kt * kWStage;
  // 4-bit tiled: 1 KiB blocks of 16 rows x 64 bytes (128 elements), lane
  // order inside, so the 64 lanes of a load read one block contiguously.
  const bool tiled = kNib && p.b_tiled;
  const int64_t w_stride = tiled ? 1024 : kWStage;  // bytes between a row's stages
  const uint8_t* w_ptr[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j)
    w_ptr[j] = tiled ? Be + (wrow[j] >> 4) * 16 * w_bytes + (lane >> 4) * 256 + (wrow[j] & 15) * 16
                     : Be + wrow[j] * w_bytes + lane_off_w;

  // fp8 weight-scale row of each lane's weight rows
  const int ksb = static_cast<int>(p.Kred / 128);
  const float* sb_ptr[NI] = {};
  if (kFp8) {
    const float* se = p.b_scale + static_cast<int64_t>(e) * (p.Nout / 128) * ksb;
#pragma unroll
    for (int j = 0; j < NI; ++j) sb_ptr[j] = se + (wrow[j] / 128) * ksb;
  }

  // int4 group scales / zeros of the wave's 64 weight rows: one dword load per
  // lane and stage instead of 2 x NI sub-dword loads.  Virtual row v = 16 j +
  // r (r = lane % 16: the lane's row in block j).  Lanes 0-31 read the fp16
  // scales of rows v = 2 d, 2 d + 1 (d = lane), lanes 32-39 the uint4 zeros of
  // rows 8 z .. 8 z + 7 (z = lane - 32); consume() fetches each lane's values
  // with ds_bpermute.  Rows 2d / 8z start even / 8-aligned blocks of the
  // layout's rows, so the dwords are aligned.
  const uint8_t* meta_ptr = nullptr;
  int64_t meta_stride = 0;
  if constexpr (WT == WType::kInt4) {
    const int ln = lane < 32 ? lane : (lane < 40 ? lane - 32 : 0);
    const int j = lane < 32 ? ln / 8 : ln / 2;
    const int r = lane < 32 ? (2 * ln) % 16 : 8 * (ln % 2);
    int64_t row;
    if (MODE == Mode::kGemm1Silu) {
      int64_t jj = static_cast<int64_t>(nt) * (BN / 2) + (j % (NI / 2)) * 16 + r;
      if (jj >= p.N_act) jj = p.N_act - 8;
      row = gemm1_row(ACT, p.N_act, jj, j < NI / 2 ? 0 : 1);
    } else {
      row = static_cast<int64_t>(nt) * BN + j * 16 + r;
      if (row >= p.Nout) row = p.Nout - 8;
    }
    const int64_t ebase = static_cast<int64_t>(e) * (p.Kred / 128) * p.Nout + row;
    if (lane < 32) {
      meta_ptr = reinterpret_cast<const uint8_t*>(p.b_gscale) + 2 * ebase;
      meta_stride = 2 * p.Nout;
    } else {
      meta_ptr = p.b_zero + (ebase >> 1);
      meta_stride = p.Nout / 2;
    }
  }

  f32x4_t acc[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto load = [&](int kt, Stage<WT>& S) {
    const int64_t woff = static_cast<int64_t>(kt) * w_stride;
    const uint8_t* ap = a_ptr + static_cast<int64_t>(kt) * kElems * 2 + lane_off_a;
    if constexpr (WT == WType::kBf16) {
      S.a = gload32(ap);
#pragma unroll
      for (int j = 0; j < NI; ++j) S.b[j] = gload32(w_ptr[j] + woff);
    } else if constexpr (WT == WType::kFp8) {
#pragma unroll
      for (int q = 0; q < 4; ++q) S.a[q] = *reinterpret_cast<const i32x4_t*>(ap + 16 * q);
#pragma unroll
      for (int j = 0; j < NI; ++j) S.b[j] = gload32(w_ptr[j] + woff);
#pragma unroll
      for (int j = 0; j < NI; ++j) S.sb[j] = sb_ptr[j][kt];
    } else if constexpr (kMx) {
#pragma unroll
      for (int q = 0; q < 4; ++q) S.a[q] = *reinterpret_cast<const i32x4_t*>(ap + 16 * q);
#pragma unroll
      for (int j = 0; j < NI; ++j) S.b[j] = *reinterpret_cast<const i32x4_t*>(w_ptr[j] + woff);
      // this lane's 32 elements are scale block 4 kt + lane / 16 of its row
      const int64_t nblk = p.Kred / 32;
#pragma unroll
      for (int j = 0; j < NI; ++j)
        S.sx[j] = p.b_mxscale[(static_cast<int64_t>(e) * p.Nout + wrow[j]) * nblk + 4 * kt + (lane >> 4)];
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) S.a[q] = *reinterpret_cast<const i32x4_t*>(ap + 16 * q);
#pragma unroll
      for (int j = 0; j < NI; ++j) S.b[j] = *reinterpret_cast<const i32x4_t*>(w_ptr[j] + woff);
      // scales and zeros of group kt, fetched with the weights so that the
      // stage's loads complete together
      S.meta = 0;
      if (lane < 40) S.meta = *reinterpret_cast<const int*>(meta_ptr + kt * meta_stride);
    }
  };

  auto consume = [&](int kt, const Stage<WT>& S) {
    if constexpr (WT == WType::kBf16) {
      const bf16x8_t a0 = as_bf16x8(S.a[0], S.a[1], S.a[2], S.a[3]);
      const bf16x8_t a1 = as_bf16x8(S.a[4], S.a[5], S.a[6], S.a[7]);
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            a0, as_bf16x8(S.b[j][0], S.b[j][1], S.b[j][2], S.b[j][3]), acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            a1, as_bf16x8(S.b[j][4], S.b[j][5], S.b[j][6], S.b[j][7]), acc[j], 0, 0, 0);
      }
    } else if constexpr (WT == WType::kFp8) {
      // quantize this lane's 32 activations with the scale of their row's
      // 128-group (the group spans the 4 lane groups holding the row)
      float x[32];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = static_cast<uint32_t>(S.a[q][i]);
          x[8 * q + 2 * i] = __uint_as_float(w << 16);
          x[8 * q + 2 * i + 1] = __uint_as_float(w & 0xffff0000u);
        }
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
      amax = fmaxf(amax, __shfl_xor(amax, 16, kWave));
      amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));
      const float sa_row = fmaxf(amax, kFp8Eps) / kFp8Max;  // scale of row lane%16
      const float inv = 1.0f / sa_row;
      // x / sa_row and the e4m3 codes exactly as the quant pass computes them
      int qa[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        qa[i] = static_cast<int>(pack_e4m3x4(fp8_qdiv(x[4 * i], sa_row, inv), fp8_qdiv(x[4 * i + 1], sa_row, inv),
                                             fp8_qdiv(x[4 * i + 2], sa_row, inv), fp8_qdiv(x[4 * i + 3], sa_row, inv)));
      const i32x8_t a = i32x8_t{qa[0], qa[1], qa[2], qa[3], qa[4], qa[5], qa[6], qa[7]};
      // output rows of this lane are 4*(lane/16) + r: fetch their scales
      float sa[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sa[r] = __shfl(sa_row, (lane >> 4) * 4 + r, kWave);
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        f32x4_t t = {0.f, 0.f, 0.f, 0.f};
        t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, S.b[j], t, 0, 0, 0, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][r] += t[r] * (sa[r] * S.sb[j]);
      }
    } else if constexpr (kMx) {
      // e2m1 -> bf16 with the block scale folded in (hardware conversion,
      // exact: e2m1 x 2^k fits bf16), then plain bf16 MFMAs.  Dword d of the
      // lane's 16 bytes holds its elements 8d..8d+7, low nibble first -- the
      // same order as the activations in S.a[d].
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const unsigned ex = S.sx[j];
        const float sc = ex == 0 ? 0x1p-127f : (ex == 255 ? __builtin_nanf("") : __uint_as_float(ex << 23));
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const unsigned wv = static_cast<unsigned>(S.b[j][d]);
          const int b0 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wv, sc, 0));
          const int b1 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wv, sc, 1));
          const int b2 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wv, sc, 2));
          const int b3 = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wv, sc, 3));
          const i32x4_t av = S.a[d];
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[0], av[1], av[2], av[3]),
                                                           as_bf16x8(b0, b1, b2, b3), acc[j], 0, 0, 0);
        }
      }
    }
    // (int4 stages are consumed inline by the main loop below)
  };

  // split-K range over stages, then interleaved over the 4 waves, PIPE
  // stages in flight per wave
  const int per_split = (nk + p.splits - 1) / p.splits;
  const int k_beg = split * per_split;
  const int k_end = min(nk, k_beg + per_split);
  if constexpr (PIPE == 2) {
    Stage<WT> s0, s1;
    int kt = k_beg + kw;
    if (kt < k_end) load(kt, s0);
    while (kt < k_end) {
      const int k1 = kt + kWaves;
      if (k1 < k_end) load(k1, s1);
      if constexpr (decode_prio<WT>() > 0) __builtin_amdgcn_s_setprio(decode_prio<WT>());
      consume(kt, s0);
      if constexpr (decode_prio<WT>() > 0) __builtin_amdgcn_s_setprio(0);
      if (k1 >= k_end) break;
      const int k2 = k1 + kWaves;
      if (k2 < k_end) load(k2, s0);
      if constexpr (decode_prio<WT>() > 0) __builtin_amdgcn_s_setprio(decode_prio<WT>());
      consume(k1, s1);
      if constexpr (decode_prio<WT>() > 0) __builtin_amdgcn_s_setprio(0);
      kt = k2;
    }
  } else if constexpr (WT == WType::kInt4) {
    // One stage of registers, reloaded piecewise as soon as each piece has
    // been consumed: the scale / zero dword right after it is spread with
    // ds_bpermute, each weight row block right after its MFMAs, the
    // activations (an L2 hit) after the last MFMA.  The next stage's loads then overlap
    // this stage's arithmetic without a second set of stage registers (which
    // would cost a wave per SIMD of occupancy).
    Stage<WT> S;
    int kt = k_beg + kw;
    const int64_t a_step = static_cast<int64_t>(kWaves) * kElems * 2;  // activation bytes per step
    const int64_t w_step = static_cast<int64_t>(kWaves) * w_stride;
    const uint8_t* ap = a_ptr + static_cast<int64_t>(kt) * kElems * 2 + lane_off_a;
    const uint8_t* mp = meta_ptr + kt * meta_stride;
    int64_t woff = static_cast<int64_t>(kt) * w_stride;
    if (kt < k_end) load(kt, S);
    const int r16 = lane & 15;
    const bf16x8_t ones = as_bf16x8(0x3f803f80, 0x3f803f80, 0x3f803f80, 0x3f803f80);
    // One step: consume stage kt, reloading the next stage's pieces as they
    // free up (MORE) or not (the last step).  Peeled so that no load sits
    // under a branch: the compiler then counts the loads exactly, and a
    // step's first ds_bpermute waits only for the scale / zero dword.
    auto step = [&](auto more_tag) {
      constexpr bool MORE = decltype(more_tag)::value;
      if constexpr (decode_prio<WT>() > 0) __builtin_amdgcn_s_setprio(decode_prio<WT>());
      ap += a_step;
      mp += kWaves * meta_stride;
      woff += w_step;
      unsigned sw[NI], zw[NI];
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        sw[j] = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(4 * (8 * j + (r16 >> 1)), S.meta));
        zw[j] = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(4 * (32 + 2 * j + (r16 >> 3)), S.meta));
      }
      // every lane loads (lanes 40-63 repeat a valid zero dword that no
      // ds_bpermute reads)
      if constexpr (MORE) S.meta = *reinterpret_cast<const int*>(mp);
      // activations of nibble dword d, permuted to the (j, j+4) pairing
      bf16x8_t a[4];
      f32x4_t xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int x01 = S.a[d][0], x23 = S.a[d][1], x45 = S.a[d][2], x67 = S.a[d][3];
        a[d] = as_bf16x8(__builtin_amdgcn_perm(x45, x01, 0x05040100), __builtin_amdgcn_perm(x45, x01, 0x07060302),
                         __builtin_amdgcn_perm(x67, x23, 0x05040100), __builtin_amdgcn_perm(x67, x23, 0x07060302));
        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d], ones, xs, 0, 0, 0);
      }
      // tiled weights: the next stage's activations (its first use) as soon
      // as the registers are free, then its weights block by block below;
      // row-major weights: the activations last (measured faster there)
      if constexpr (MORE) {
        if (tiled) {
#pragma unroll
          for (int q = 0; q < 4; ++q) S.a[q] = *reinterpret_cast<const i32x4_t*>(ap + 16 * q);
        }
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const unsigned wv = static_cast<unsigned>(S.b[j][d]);
          const int b0 = static_cast<int>((wv & 0x000f000fu) | 0x43004300u);
          const int b1 = static_cast<int>(((wv >> 4) & 0x000f000fu) | 0x43004300u);
          const int b2 = static_cast<int>(((wv >> 8) & 0x000f000fu) | 0x43004300u);
          const int b3 = static_cast<int>(((wv >> 12) & 0x000f000fu) | 0x43004300u);
          t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d], as_bf16x8(b0, b1, b2, b3), t, 0, 0, 0);
        }
        if constexpr (MORE) S.b[j] = *reinterpret_cast<const i32x4_t*>(w_ptr[j] + woff);
        const float sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>((r16 & 1) ? (sw[j] >> 16) : (sw[j] & 0xffffu))));
        const float z = static_cast<float>((zw[j] >> (4 * (r16 & 7))) & 15u);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][r] += sc * (t[r] - (128.0f + z) * xs[r]);
      }
      if constexpr (MORE) {
        if (!tiled) {
#pragma unroll
          for (int q = 0; q < 4; ++q) S.a[q] = *reinterpret_cast<const i32x4_t*>(ap + 16 * q);
        }
      }
      if constexpr (decode_prio<WT>() > 0) __builtin_amdgcn_s_setprio(0);
    };
    for (; kt + kWaves < k_end; kt += kWaves) step(std::true_type{});
    if (kt < k_end) step(std::false_type{});
  } else {
    for (int kt = k_beg + kw; kt < k_end; kt += kWaves) {
      Stage<WT> s0;
      load(kt, s0);
      if constexpr (decode_prio<WT>() > 0) __builtin_amdgcn_s_setprio(decode_prio<WT>());
      consume(kt, s0);
      if constexpr (decode_prio<WT>() > 0) __builtin_amdgcn_s_setprio(0);
    }
  }

  // ---- reduce the 4 waves' partials
#pragma unroll
  for (int j = 0; j < NI; ++j) red[rb][kw][j][lane] = acc[j];
  __syncthreads();
  if (kw != 0) return;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    f32x4_t v = red[rb][0][j][lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      f32x4_t u = red[rb][w][j][lane];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] += u[r];
    }
    acc[j] = v;
  }

  const int col16 = lane & 15;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int rr = (lane >> 4) * 4 + r;
    if (rr >= n_rows) continue;
    const int s = slot_of(rr);
    const float g = p.gamma ? (TINY ? p.tiny_w[s] : p.gate_scal[s]) : 1.0f;
    if (MODE == Mode::kGemm1Silu) {
      uint16_t* act = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(s) * p.N_act;
#pragma unroll
      for (int j = 0; j < NI / 2; ++j) {
        const int64_t col = static_cast<int64_t>(nt) * (BN / 2) + j * 16 + col16;
        if (col >= p.N_act) continue;
        float gb, ub;
        gemm1_bias<ACT>(p, e, col, gb, ub);
        act[col] = f32_to_bf16(gemm1_act<ACT>(p, acc[j][r], acc[j + NI / 2][r], gb, ub, g));
      }
    } else {
      float* y = static_cast<float*>(p.out) + split * p.out_split_stride +
                 static_cast<int64_t>(s) * p.Nout;
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int64_t col = static_cast<int64_t>(nt) * BN + j * 16 + col16;
        if (col < p.Nout) {
          const float b = (p.bias && split == 0) ? p.bias[static_cast<int64_t>(e) * p.Nout + col] : 0.f;
          y[col] = (acc[j][r] + b) * g;
        }
      }
    }
  }
}

// int4 decode, row split: the workgroup's 4 waves each own one 64-row block
// of the weights over the whole reduction range (of this split), all on the
// same stage at a time, so the activation stage is loaded once per workgroup
// instead of once per wave: each wave brings a quarter of it two stages ahead,
// through registers into a 3-slot LDS ring published by one barrier per
// stage.  All global loads are ordinary compiler-tracked loads.  Weights,
// scales / zeros and the arithmetic are the row-block kernel's (one stage of
// weight registers reloaded piecewise).
// PAIR: a workgroup takes a pair of the routing's 16-slot tiles, the
// expert's tiles 2i and 2i + 1 (32 rows, 8 KiB of activations per stage), so
// every weight fragment feeds two MFMA row halves and the workgroup of an odd
// tile exits: an expert with 17-32 slots streams its weights once instead of
// twice.  Padding rows re-read the tile's first row (coalesced with it by the
// load instruction).  It needs ~160 VGPRs (3 waves per SIMD instead of 4), so
// it is taken when the experts average >= 24 slots (Mixtral W4A16 M=256: 535
// -> 450-465 µs; at M=64, ~16 +- 4 slots, the single tiles would pay the
// second half and the occupancy: 3-5% slower).
constexpr int kRsBlocks = 4;  // row blocks (= waves) per workgroup
constexpr int kRsThreads = 64 * kRsBlocks;
static_assert(kRsBlocks == 1 || kRsBlocks == 2 || kRsBlocks == 4, "row blocks per workgroup");
constexpr int kRsPitch = 256 + 16;  // LDS bytes per activation row (padded against bank conflicts)
constexpr int kRsPairMinSlots = 24;  // mean slots per expert from which tiles are paired

template <Mode MODE, int ACT, bool PAIR>
__global__ __launch_bounds__(kRsThreads, PAIR ? 2 : 16 / kRsBlocks) void gemm_decode_int4_rs_kernel(GemmParams p) {
  constexpr int H = PAIR ? 2 : 1;                      // 16-row halves
  constexpr int kRsRows = H * BM;                      // activation rows of the workgroup
  constexpr int kRsPieces = kRsRows / (4 * kRsBlocks);  // activation loads per lane and stage
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[3][kRsRows * kRsPitch];
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wid = __builtin_amdgcn_readfirstlane(tid / kWave);
  // workgroup -> (split, tile, group of 4 row blocks), XCD-contiguous as in
  // gemm_decode_kernel (row blocks fastest when a tile has <= 128 of them)
  const int gy = gridDim.y;
  const int ntl = *p.n_tiles;
  const int live = ntl * gy * gridDim.z;
  const int b = blockIdx.x + gridDim.x * (blockIdx.y + gy * blockIdx.z);
  if (b >= live) return;
  const int L = xcd_remap(b, live);
  const int split = L / (gy * ntl);
  int mt, ntw;
  if (gy * kRsBlocks <= 128) {
    ntw = L % gy;
    mt = (L / gy) % ntl;
  } else {
    mt = L % ntl;
    ntw = (L / ntl) % gy;
  }
  const int nt = ntw * kRsBlocks + wid;  // this wave's 64-row block
  const int tm = p.tile_map[mt];
  if (PAIR && ((tm >> 16) & 1)) return;  // the odd tile of a pair: computed with the even one
  const int e = tm & 0xffff;
  const int row_beg = p.offs_raw[e] + (tm >> 16) * BM;
  const int n_rows = min(p.offs_raw[e + 1], row_beg + kRsRows) - row_beg;

  // activation rows: piece h of this lane is row (kRsRows / kRsBlocks) wid +
  // 4 h + lane / 16 (16 bytes of its 256-byte stage slice); fragments are
  // read as the row-block kernel loads them (lane -> row 16 half + lane % 16,
  // bytes 64 (lane / 16) .. + 63)
  const uint8_t* a_src[kRsPieces];
  int a_dst[kRsPieces];
#pragma unroll
  for (int h = 0; h < kRsPieces; ++h) {
    const int ar = (kRsRows / kRsBlocks) * wid + 4 * h + (lane >> 4);
    const int as = row_beg + (ar < n_rows ? ar : 0);
    const int64_t a_row = MODE == Mode::kGemm1Silu ? p.topk_indx[as] / p.top_k : as;
    a_src[h] = p.A + a_row * p.Kred * 2 + (lane & 15) * 16;
    a_dst[h] = ar * kRsPitch + (lane & 15) * 16;
  }
  const int a_frag = (lane & 15) * kRsPitch + (lane >> 4) * 64;  // half 1: + 16 rows

  const int64_t w_bytes = p.Kred / 2;
  const int nk = static_cast<int>(p.Kred / 128);
  const uint8_t* Be = p.B + static_cast<int64_t>(e) * p.Nout * w_bytes;
  int64_t wrow[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    int64_t r;
    if (MODE == Mode::kGemm1Silu) {
      int64_t jj = static_cast<int64_t>(nt) * (BN / 2) + (j % (NI / 2)) * 16 + (lane & 15);
      if (jj >= p.N_act) jj = p.N_act - 1;
      r = gemm1_row(ACT, p.N_act, jj, j < NI / 2 ? 0 : 1);
    } else {
      r = static_cast<int64_t>(nt) * BN + j * 16 + (lane & 15);
      if (r >= p.Nout) r = p.Nout - 1;
    }
    wrow[j] = r;
  }
  const bool tiled = p.b_tiled;
  const int64_t w_stride = tiled ? 1024 : 64;  // bytes between a row's stages
  const uint8_t* w_ptr[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j)
    w_ptr[j] = tiled ? Be + (wrow[j] >> 4) * 16 * w_bytes + (lane >> 4) * 256 + (wrow[j] & 15) * 16
                     : Be + wrow[j] * w_bytes + (lane >> 4) * 16;
  // group scales (lanes 0-31) / zeros (lanes 32-39) of the wave's rows, one
  // dword per lane and stage (the row-block kernel's scheme)
  const uint8_t* meta_ptr;
  int64_t meta_stride;
  {
    const int ln = lane < 32 ? lane : (lane < 40 ? lane - 32 : 0);
    const int j = lane < 32 ? ln / 8 : ln / 2;
    const int r = lane < 32 ? (2 * ln) % 16 : 8 * (ln % 2);
    int64_t row;
    if (MODE == Mode::kGemm1Silu) {
      int64_t jj = static_cast<int64_t>(nt) * (BN / 2) + (j % (NI / 2)) * 16 + r;
      if (jj >= p.N_act) jj = p.N_act - 8;
      row = gemm1_row(ACT, p.N_act, jj, j < NI / 2 ? 0 : 1);
    } else {
      row = static_cast<int64_t>(nt) * BN + j * 16 + r;
      if (row >= p.Nout) row = p.Nout - 8;
    }
    const int64_t ebase = static_cast<int64_t>(e) * (p.Kred / 128) * p.Nout + row;
    if (lane < 32) {
      meta_ptr = reinterpret_cast<const uint8_t*>(p.b_gscale) + 2 * ebase;
      meta_stride = 2 * p.Nout;
    } else {
      meta_ptr = p.b_zero + (ebase >> 1);
      meta_stride = p.Nout / 2;
    }
  }

  f32x4_t acc[H][NI];
#pragma unroll
  for (int h = 0; h < H; ++h)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[h][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int per_split = (nk + p.splits - 1) / p.splits;
  const int k_beg = min(nk, split * per_split);
  const int n = min(nk, k_beg + per_split) - k_beg;  // stages of this split (same for every wave)
  i32x4_t an[kRsPieces];  // this lane's pieces of a later activation stage
  i32x4_t wb[NI];
  int meta = 0;
  int64_t woff = static_cast<int64_t>(k_beg) * w_stride;
  const uint8_t* mp = meta_ptr + k_beg * meta_stride;
  if (n > 0) {
#pragma unroll
    for (int h = 0; h < kRsPieces; ++h) {
      an[h] = *reinterpret_cast<const i32x4_t*>(a_src[h] + static_cast<int64_t>(k_beg) * 256);
      *reinterpret_cast<i32x4_t*>(&a_lds[0][a_dst[h]]) = an[h];
      if (n > 1) an[h] = *reinterpret_cast<const i32x4_t*>(a_src[h] + static_cast<int64_t>(k_beg + 1) * 256);
    }
#pragma unroll
    for (int j = 0; j < NI; ++j) wb[j] = *reinterpret_cast<const i32x4_t*>(w_ptr[j] + woff);
    meta = *reinterpret_cast<const int*>(mp);  // every lane: see the row-block kernel
  }
  __syncthreads();
  const int r16 = lane & 15;
  const bf16x8_t ones = as_bf16x8(0x3f803f80, 0x3f803f80, 0x3f803f80, 0x3f803f80);
  // Every global load of the loop is unconditional, the stage index clamped
  // to the split's last stage (the last iterations re-read it: L2 hits):
  // under a branch the compiler waited for all outstanding loads (the
  // activation piece of stage kt + 2 included) before the first ds_bpermute.
  const int k_last = k_beg + n - 1;
  for (int i = 0; i < n; ++i) {
    const int kt = k_beg + i;
    const bool more = i + 1 < n;
    // publish stage kt + 1 (its slot was last read at stage kt - 2), fetch
    // this lane's piece of stage kt + 2
#pragma unroll
    for (int h = 0; h < kRsPieces; ++h) {
      if (more) *reinterpret_cast<i32x4_t*>(&a_lds[(i + 1) % 3][a_dst[h]]) = an[h];
      an[h] = *reinterpret_cast<const i32x4_t*>(a_src[h] + static_cast<int64_t>(min(kt + 2, k_last)) * 256);
    }
    const int k1 = min(kt + 1, k_last);
    woff = static_cast<int64_t>(k1) * w_stride;
    mp = meta_ptr + k1 * meta_stride;
    unsigned sw[NI], zw[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      sw[j] = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(4 * (8 * j + (r16 >> 1)), meta));
      zw[j] = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(4 * (32 + 2 * j + (r16 >> 3)), meta));
    }
    // every lane loads (lanes 40-63 repeat a valid zero dword): under a
    // lane-dependent branch the compiler waited for all outstanding loads,
    // the activation piece of stage kt + 2 included, before the ds_bpermutes
    meta = *reinterpret_cast<const int*>(mp);
    // activations of stage kt for both row halves, permuted to the (j, j+4)
    // nibble pairing
    bf16x8_t a[H][4];
    f32x4_t xs[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
      xs[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const uint8_t* af = &a_lds[i % 3][a_frag + 16 * h * kRsPitch];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const i32x4_t v = *reinterpret_cast<const i32x4_t*>(af + 16 * d);
        a[h][d] = as_bf16x8(__builtin_amdgcn_perm(v[2], v[0], 0x05040100), __builtin_amdgcn_perm(v[2], v[0], 0x07060302),
                            __builtin_amdgcn_perm(v[3], v[1], 0x05040100), __builtin_amdgcn_perm(v[3], v[1], 0x07060302));
        xs[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[h][d], ones, xs[h], 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      f32x4_t t[H];
#pragma unroll
      for (int h = 0; h < H; ++h) t[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const unsigned wv = static_cast<unsigned>(wb[j][d]);
        const int b0 = static_cast<int>((wv & 0x000f000fu) | 0x43004300u);
        const int b1 = static_cast<int>(((wv >> 4) & 0x000f000fu) | 0x43004300u);
        const int b2 = static_cast<int>(((wv >> 8) & 0x000f000fu) | 0x43004300u);
        const int b3 = static_cast<int>(((wv >> 12) & 0x000f000fu) | 0x43004300u);
        const bf16x8_t bq = as_bf16x8(b0, b1, b2, b3);
#pragma unroll
        for (int h = 0; h < H; ++h) t[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[h][d], bq, t[h], 0, 0, 0);
      }
      wb[j] = *reinterpret_cast<const i32x4_t*>(w_ptr[j] + woff);
      const float sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>((r16 & 1) ? (sw[j] >> 16) : (sw[j] & 0xffffu))));
      const float z = static_cast<float>((zw[j] >> (4 * (r16 & 7))) & 15u);
#pragma unroll
      for (int h = 0; h < H; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[h][j][r] += sc * (t[h][r] - (128.0f + z) * xs[h][r]);
    }
    __syncthreads();  // stage kt + 1 visible; stage kt's slot free from stage kt + 2 on
  }

  // ---- epilogue: this wave's rows of both halves (the row-block kernel's,
  // without the cross-wave reduction)
  const int col16 = lane & 15;
#pragma unroll
  for (int hr = 0; hr < 4 * H; ++hr) {
    const int h = hr >> 2, r = hr & 3;
    const int rr = 16 * h + (lane >> 4) * 4 + r;
    if (rr >= n_rows) continue;
    const int s = row_beg + rr;
    const float g = p.gamma ? p.gate_scal[s] : 1.0f;
    if (MODE == Mode::kGemm1Silu) {
      uint16_t* act = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(s) * p.N_act;
#pragma unroll
      for (int j = 0; j < NI / 2; ++j) {
        const int64_t col = static_cast<int64_t>(nt) * (BN / 2) + j * 16 + col16;
        if (col >= p.N_act) continue;
        float gb, ub;
        gemm1_bias<ACT>(p, e, col, gb, ub);
        act[col] = f32_to_bf16(gemm1_act<ACT>(p, acc[h][j][r], acc[h][j + NI / 2][r], gb, ub, g));
      }
    } else {
      float* y = static_cast<float*>(p.out) + split * p.out_split_stride + static_cast<int64_t>(s) * p.Nout;
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int64_t col = static_cast<int64_t>(nt) * BN + j * 16 + col16;
        if (col < p.Nout) {
          const float bb = (p.bias && split == 0) ? p.bias[static_cast<int64_t>(e) * p.Nout + col] : 0.f;
          y[col] = (acc[h][j][r] + bb) * g;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// int4 (tiled) decode in one launch per call: GEMM1, the activation and GEMM2
// of one 128-column slice of the intermediate dim in one workgroup.
//
// Workgroup (chunk c, tile mt) computes act[:, 128 c .. 128 c + 127] of the
// tile's slots -- GEMM1 over the whole hidden dim for 256 weight rows: 4 row
// blocks of 64 (the row-block kernel's, SiLU / GELU layout), each split over
// 4 waves by interleaved stages, i.e. the 16 waves of four row-block
// workgroups -- rounds it to bf16 into LDS (the rounding point of the
// two-launch path), then multiplies it by w2[:, 128 c .. 128 c + 127]: one
// 128-element quantization group of every w2 row, one 1 KiB tiled block per
// 16 rows.  The product goes to partial plane c, y[c][slot][0 .. K), which
// moe_sum_planes adds in fixed order.  No workgroup waits for another.
// Against GEMM1 -> act -> GEMM2 as two launches this saves a launch, the
// act round trip and the second kernel's ramp, for N / 128 partial planes of
// fp32 rows (3.7 MB for one Mixtral token): a small-batch route.
// dword 3 of a raw (untyped, stride 0) buffer descriptor on gfx950: offsets
// at or past num_records are dropped by the hardware
constexpr int kBufferDword3 = 0x00020000;
constexpr int kFzWaves = 16;
constexpr int kFzXBytes = 48 * 1024;  // LDS for the tile's x rows, later the partial sums
static_assert((kWaves - 1) * 4 * NI * kWave * 16 <= kFzXBytes, "partial sums fit the x staging LDS");
constexpr int kFzThreads = kFzWaves * kWave;
constexpr int kFzCols = 128;                      // act columns per workgroup
constexpr int kFzRowBlocks = kFzCols / (BN / 2);  // GEMM1 64-row blocks per workgroup
constexpr int kFzKw = kFzWaves / kFzRowBlocks;    // waves per row block
constexpr int kFzPitch = 2 * kFzCols + 16;        // LDS bytes per act row (padded)
constexpr int kFzBatch = 4;   // w2 16-row groups per load batch
constexpr int kFzBatchRows = 16 * kFzBatch;
static_assert(kFzBatch == 4 || kFzBatch == 8, "w2 batch: 64 or 128 rows");
static_assert(kFzKw == kWaves && kFzRowBlocks == 4, "fused int4 geometry");

// One batch of 16 kFzBatch w2 rows at the workgroup's group c: kFzBatch tiled
// blocks (16 bytes per lane each), their fp16 scales (one dword = 2 rows per
// lane) and uint4 zeros (one dword = 8 rows per lane).
struct W2Batch {
  i32x4_t w[kFzBatch];
  int sm, zm;
};

template <int ACT, bool TINY>
__global__ __launch_bounds__(kFzThreads, 1) void fused_int4_kernel(GemmParams p, GemmParams q) {
  static_assert(ACT != kActSwiglu, "int4 decode: SiLU / GELU row layout only");
  // x rows of the tile during GEMM1, then the cross-wave partial sums
  __shared__ __attribute__((aligned(16))) uint8_t xr_lds[kFzXBytes];
  auto red = reinterpret_cast<f32x4_t (*)[kFzRowBlocks][NI][kWave]>(xr_lds);
  __shared__ __attribute__((aligned(16))) uint8_t act_lds[BM * kFzPitch];
  __shared__ TinyLds tiny_lds[1];
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wid = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rb = wid % kFzRowBlocks, kw = wid / kFzRowBlocks;
  const int c = blockIdx.x, mt = blockIdx.y;

  int e, row_beg = 0, n_rows;
  if constexpr (TINY) {
    if (!tiny_route<kFzThreads>(p, mt, tiny_lds[0])) return;
    e = tiny_lds[0].info[0];
    n_rows = tiny_lds[0].info[2];
  } else {
    if (mt >= *p.n_tiles) return;
    const int tm = p.tile_map[mt];
    e = tm & 0xffff;
    row_beg = p.offs_raw[e] + (tm >> 16) * BM;
    n_rows = min(p.offs_raw[e + 1], row_beg + BM) - row_beg;
  }
  auto slot_of = [&](int r) { return TINY ? tiny_lds[0].rows[r] : row_beg + r; };
  const int r16 = lane & 15;

  // ---- GEMM1 addresses (the row-block kernel's, 64-row block nt)
  const int nt = c * kFzRowBlocks + rb;
  // the tile's x rows are staged in LDS once (n_rows K 2 <= kFzXBytes, which
  // the host guarantees): GEMM1 then issues only weight and scale loads
  {
    const int vr = static_cast<int>(p.Kred / 8);  // 16-byte pieces per row
    for (int i = tid; i < n_rows * vr; i += kFzThreads) {
      const int m = i / vr, v = i - m * vr;
      const int sm = slot_of(m);
      const int64_t xrow = (TINY ? sm : p.topk_indx[sm]) / p.top_k;
      *reinterpret_cast<i32x4_t*>(&xr_lds[(static_cast<int64_t>(m) * vr + v) * 16]) =
          *reinterpret_cast<const i32x4_t*>(p.A + (xrow * vr + v) * 16);
    }
  }
  __syncthreads();
  const int a_off = (r16 < n_rows ? r16 : 0) * static_cast<int>(p.Kred) * 2 + (lane >> 4) * 64;
  const int64_t w_bytes = p.Kred / 2;
  const int nk = static_cast<int>(p.Kred / 128);
  const uint8_t* Be = p.B + static_cast<int64_t>(e) * p.Nout * w_bytes;
  // weight rows of block j: gate rows 32 nt + 16 j + r16 (j < 2), up rows N
  // further; one per-lane base plus a uniform offset per block
  const uint8_t* w_ptr0 = Be + (static_cast<int64_t>(nt) * (BN / 2) / 16) * 16 * w_bytes + (lane >> 4) * 256 + r16 * 16;
  int64_t w_joff[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) w_joff[j] = ((j % (NI / 2)) * 16 + (j < NI / 2 ? 0 : p.N_act)) * w_bytes;
  // scales (lanes 0-31: rows 2 d, 2 d + 1 of the virtual 16 j + r order) and
  // zeros (lanes 32-39: rows 8 z .. 8 z + 7), one dword per lane and stage:
  // element index mrow + kt N_out of the expert's [K / 128][N_out] arrays
  // (uniform bases, a 32-bit per-lane index: no 64-bit pointer per lane)
  int mrow;
  {
    const int ln = lane < 32 ? lane : (lane < 40 ? lane - 32 : 0);
    const int j = lane < 32 ? ln / 8 : ln / 2;
    const int r = lane < 32 ? (2 * ln) % 16 : 8 * (ln % 2);
    const int64_t jj = static_cast<int64_t>(nt) * (BN / 2) + (j % (NI / 2)) * 16 + r;
    mrow = static_cast<int>(gemm1_row(ACT, p.N_act, jj, j < NI / 2 ? 0 : 1));
  }
  const int64_t mbase = static_cast<int64_t>(e) * nk * p.Nout;
  const uint16_t* ms = p.b_gscale + mbase;
  const uint8_t* mz = p.b_zero + (mbase >> 1);
  const int nout1 = static_cast<int>(p.Nout);

  // ---- GEMM1: stages kw, kw + 4, ...; one stage of registers, reloaded
  // piecewise as soon as each piece is consumed (scale / zero dword after its
  // ds_bpermutes, each weight block after its MFMAs, the activations -- L2
  // hits -- after the last MFMA), so the next stage's loads overlap this
  // stage's arithmetic
  const bf16x8_t ones = as_bf16x8(0x3f803f80, 0x3f803f80, 0x3f803f80, 0x3f803f80);
  f32x4_t acc[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // one unconditional meta load per lane (lanes 40-63 re-read a zero dword)
  auto meta_at = [&](int kt) {
    const int mi = mrow + kt * nout1;
    return *reinterpret_cast<const int*>(lane < 32 ? reinterpret_cast<const uint8_t*>(ms + mi) : mz + (mi >> 1));
  };
  {
    int kt = kw;
    i32x4_t av[4], wb[NI];
    int meta = 0;
    if (kt < nk) {
#pragma unroll
      for (int d = 0; d < 4; ++d) av[d] = *reinterpret_cast<const i32x4_t*>(&xr_lds[a_off + kt * 256 + 16 * d]);
#pragma unroll
      for (int j = 0; j < NI; ++j) wb[j] = *reinterpret_cast<const i32x4_t*>(w_ptr0 + w_joff[j] + static_cast<int64_t>(kt) * 1024);
      meta = meta_at(kt);
    }
    // peeled last step: no load sits under a branch, so the compiler's waits
    // before the scale / zero ds_bpermutes and each weight block count exactly
    auto step = [&](auto more_tag) {
      constexpr bool MORE = decltype(more_tag)::value;
      const int kn = kt + kFzKw;
      unsigned sw[NI], zw[NI];
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        sw[j] = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(4 * (8 * j + (r16 >> 1)), meta));
        zw[j] = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(4 * (32 + 2 * j + (r16 >> 3)), meta));
      }
      if constexpr (MORE) meta = meta_at(kn);
      bf16x8_t a[4];
      f32x4_t xs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int x01 = av[d][0], x23 = av[d][1], x45 = av[d][2], x67 = av[d][3];
        a[d] = as_bf16x8(__builtin_amdgcn_perm(x45, x01, 0x05040100), __builtin_amdgcn_perm(x45, x01, 0x07060302),
                         __builtin_amdgcn_perm(x67, x23, 0x05040100), __builtin_amdgcn_perm(x67, x23, 0x07060302));
        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d], ones, xs, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const unsigned wv = static_cast<unsigned>(wb[j][d]);
          const int b0 = static_cast<int>((wv & 0x000f000fu) | 0x43004300u);
          const int b1 = static_cast<int>(((wv >> 4) & 0x000f000fu) | 0x43004300u);
          const int b2 = static_cast<int>(((wv >> 8) & 0x000f000fu) | 0x43004300u);
          const int b3 = static_cast<int>(((wv >> 12) & 0x000f000fu) | 0x43004300u);
          t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[d], as_bf16x8(b0, b1, b2, b3), t, 0, 0, 0);
        }
        if constexpr (MORE) wb[j] = *reinterpret_cast<const i32x4_t*>(w_ptr0 + w_joff[j] + static_cast<int64_t>(kn) * 1024);
        const float sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>((r16 & 1) ? (sw[j] >> 16) : (sw[j] & 0xffffu))));
        const float z = static_cast<float>((zw[j] >> (4 * (r16 & 7))) & 15u);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][r] += sc * (t[r] - (128.0f + z) * xs[r]);
      }
      if constexpr (MORE) {
#pragma unroll
        for (int d = 0; d < 4; ++d) av[d] = *reinterpret_cast<const i32x4_t*>(&xr_lds[a_off + kn * 256 + 16 * d]);
      }
    };
    for (; kt + kFzKw < nk; kt += kFzKw) step(std::true_type{});
    if (kt < nk) step(std::false_type{});
  }

  // ---- GEMM2 operands: the wave's row batches b = wid, wid + 16, ...;
  // the first batch is requested before the GEMM1 reduction
  const int64_t K2 = q.Nout;
  const int64_t w2_bytes = q.Kred / 2;
  const int n_blk = static_cast<int>(K2 / kFzBatchRows);
  const int64_t grp = static_cast<int64_t>(e) * (q.Kred / 128) + c;  // (expert, quant group)
  const uint8_t* B2 = q.B + static_cast<int64_t>(e) * K2 * w2_bytes + static_cast<int64_t>(c) * 1024 +
                      (lane >> 4) * 256 + r16 * 16;
  const uint16_t* s2 = q.b_gscale + grp * K2;
  const uint8_t* z2 = q.b_zero + (grp * K2) / 2;
  auto load2 = [&](int b, W2Batch& W) {
#pragma unroll
    for (int i = 0; i < kFzBatch; ++i)
      W.w[i] = *reinterpret_cast<const i32x4_t*>(B2 + static_cast<int64_t>(b * kFzBatch + i) * 16 * w2_bytes);
    // unconditional loads (surplus lanes re-read a valid dword): no branch
    // between the batch's loads and the waits for the previous batch
    W.sm = *reinterpret_cast<const int*>(s2 + kFzBatchRows * b + 2 * (lane % (kFzBatchRows / 2)));
    W.zm = *reinterpret_cast<const int*>(z2 + kFzBatchRows / 2 * b + 4 * (lane % (kFzBatchRows / 8)));

  };
  W2Batch W0, W1;
  int b = wid;
  if (b < n_blk) load2(b, W0);

  // GEMM2 output slots of this lane (tile rows 4 (lane / 16) + r) and their
  // gammas, loaded before the barriers below, which wait for them: the GEMM2
  // loop's waits then need not cover them
  int ys[4];
  float yg[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = (lane >> 4) * 4 + r;
    ys[r] = m < n_rows ? slot_of(m) : -1;
    yg[r] = (ys[r] >= 0 && q.gamma) ? (TINY ? q.tiny_w[ys[r]] : q.gate_scal[ys[r]]) : 1.0f;
  }

  // ---- GEMM1 reduction over the 4 waves of a row block, activation -> LDS
  __syncthreads();  // every wave has read its last x stage: the LDS takes the partial sums
  if (kw > 0) {
#pragma unroll
    for (int j = 0; j < NI; ++j) red[kw - 1][rb][j][lane] = acc[j];
  }
  __syncthreads();
  if (kw == 0) {
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int w = 0; w < kFzKw - 1; ++w) {
        const f32x4_t u = red[w][rb][j][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][r] += u[r];
      }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = (lane >> 4) * 4 + r;
      float g = 1.0f;
      if (m < n_rows && p.gamma) {
        const int s = slot_of(m);
        g = TINY ? p.tiny_w[s] : p.gate_scal[s];
      }
#pragma unroll
      for (int j = 0; j < NI / 2; ++j) {
        const uint16_t v = m < n_rows ? f32_to_bf16(gemm1_act<ACT>(p, acc[j][r], acc[j + NI / 2][r], 0.f, 0.f, g)) : 0;
        *reinterpret_cast<uint16_t*>(&act_lds[m * kFzPitch + 2 * (rb * (BN / 2) + j * 16 + r16)]) = v;
      }
    }
  }
  __syncthreads();

  // ---- GEMM2: A = the tile's act slice (lane: row r16, elements 32 (lane /
  // 16) .. + 31, permuted to the nibble pairing), shared by every batch
  bf16x8_t a2[4];
  f32x4_t xs2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const i32x4_t v = *reinterpret_cast<const i32x4_t*>(&act_lds[r16 * kFzPitch + (lane >> 4) * 64 + 16 * d]);
    a2[d] = as_bf16x8(__builtin_amdgcn_perm(v[2], v[0], 0x05040100), __builtin_amdgcn_perm(v[2], v[0], 0x07060302),
                      __builtin_amdgcn_perm(v[3], v[1], 0x05040100), __builtin_amdgcn_perm(v[3], v[1], 0x07060302));
    xs2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[d], ones, xs2, 0, 0, 0);
  }
  // y stores go through a buffer descriptor over the call's planes: rows of
  // the tile without a slot get an out-of-range offset, which the hardware
  // drops -- no branch around the stores (a branch there makes the compiler
  // wait for the next batch's loads before storing)
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
      q.out, 0, static_cast<int>(static_cast<int64_t>(q.splits) * q.out_split_stride * 4), kBufferDword3);
  uint32_t yoff[4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    yoff[r] = ys[r] >= 0 ? static_cast<uint32_t>((c * q.out_split_stride + static_cast<int64_t>(ys[r]) * K2) * 4)
                         : 0x80000000u;
  auto consume2 = [&](int bb, const W2Batch& W) {
#pragma unroll
    for (int i = 0; i < kFzBatch; ++i) {
      f32x4_t t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const unsigned wv = static_cast<unsigned>(W.w[i][d]);
        const int b0 = static_cast<int>((wv & 0x000f000fu) | 0x43004300u);
        const int b1 = static_cast<int>(((wv >> 4) & 0x000f000fu) | 0x43004300u);
        const int b2 = static_cast<int>(((wv >> 8) & 0x000f000fu) | 0x43004300u);
        const int b3 = static_cast<int>(((wv >> 12) & 0x000f000fu) | 0x43004300u);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[d], as_bf16x8(b0, b1, b2, b3), t, 0, 0, 0);
      }
      // row 16 i + r16 of the batch: scale half r16 % 2 of lane 8 i + r16 / 2,
      // zero nibble r16 % 8 of lane 2 i + r16 / 8
      const unsigned sw = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(4 * (8 * i + (r16 >> 1)), W.sm));
      const unsigned zw = static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(4 * (2 * i + (r16 >> 3)), W.zm));
      const float sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>((r16 & 1) ? (sw >> 16) : (sw & 0xffffu))));
      const float z = static_cast<float>((zw >> (4 * (r16 & 7))) & 15u);
      const int64_t col = static_cast<int64_t>(bb) * kFzBatchRows + i * 16 + r16;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sc * (t[r] - (128.0f + z) * xs2[r]) * yg[r]), yr,
                                              static_cast<int>(yoff[r] + 4 * static_cast<uint32_t>(col)), 0, 0);
    }
  };
  while (b < n_blk) {
    const int b1 = b + kFzWaves;
    if (b1 < n_blk) load2(b1, W1);
    consume2(b, W0);
    if (b1 >= n_blk) break;
    const int b2 = b1 + kFzWaves;
    if (b2 < n_blk) load2(b2, W0);
    consume2(b1, W1);
    b = b2;
  }
}


}  // namespace decode

// Row blocks per workgroup by format (measured: two for fp8, one otherwise).
constexpr int decode_row_blocks(WType wt) { return wt == WType::kFp8 ? 2 : 1; }
static_assert(decode_row_blocks(WType::kBf16) >= 1 && decode_row_blocks(WType::kBf16) <= decode::kMaxRB &&
                  decode_row_blocks(WType::kFp8) >= 1 && decode_row_blocks(WType::kFp8) <= decode::kMaxRB &&
                  decode_row_blocks(WType::kInt4) >= 1 && decode_row_blocks(WType::kInt4) <= decode::kMaxRB &&
                  decode_row_blocks(WType::kMxfp4) >= 1 && decode_row_blocks(WType::kMxfp4) <= decode::kMaxRB,
              "decode row blocks out of range");

// int4 with the align launch and many tiles: the row-split kernel (one
// activation stage per workgroup) instead of the row-block kernel.  Measured
// on Mixtral W4A16 (tiled): M=64 (15 tiles) 254 -> 244 us; at M=4 / 16 (<= 9
// tiles) its 4x coarser workgroups balance worse: 13% / 5% slower there.
constexpr int kRsMinTiles = 14;
// row blocks per workgroup of the int4 row-split kernel for a grid of
// max_tiles expert tiles, 0 when the row-block kernel runs
int decode_int4_row_split(int64_t max_tiles) {
  return max_tiles >= kRsMinTiles ? decode::kRsBlocks : 0;
}

// Whether the row-split kernel pairs tiles: slots estimated from the tile
// bound (max_tiles = E - 1 + ceil((slots - E + 1) / 16), so >= the slots / 16)
bool decode_int4_pair(int64_t max_tiles, int E) {
  const int64_t slots_est = (max_tiles - (E - 1)) * decode::BM;
  return slots_est >= static_cast<int64_t>(decode::kRsPairMinSlots) * E;
}

// Whether a call with `slots` top-k slots and hidden size K fits the one-launch
// int4 kernel's LDS staging of a tile's x rows (at most min(16, slots) rows).
bool fused_int4_fits(int64_t slots, int64_t K) {
  const int64_t rows = slots < decode::BM ? slots : decode::BM;
  return rows * K * 2 <= decode::kFzXBytes;
}

// One launch of fused_int4_kernel: p = GEMM1 (x, w13, routing: tile map or
// the tiny-batch top-k ids), q = GEMM2 (w2, gammas, bias, y planes).
int launch_fused_int4(const GemmParams& p, const GemmParams& q, hipStream_t s) {
  if (p.max_tiles <= 0) return FMOE_OK;
  if (p.N_act % decode::kFzCols != 0 || q.Nout % 128 != 0 || p.act == kActSwiglu || p.bias || q.bias ||
      q.splits != p.N_act / decode::kFzCols || static_cast<int64_t>(q.splits) * q.out_split_stride * 4 >= (int64_t(1) << 31) ||
      !fused_int4_fits(q.out_split_stride / q.Nout, p.Kred))
    return fmoe_host::fail(FMOE_ERR_UNSUPPORTED,
                           "fused int4 decode: N %% 128, K %% 128, SiLU / GELU, no bias, N / 128 planes < 2 GiB, x rows in LDS");
  const dim3 g(static_cast<unsigned>(p.N_act / decode::kFzCols), static_cast<unsigned>(p.max_tiles));
  const dim3 b(decode::kFzThreads);
  const bool tiny = p.tiny_ids != nullptr;
  if (p.act == kActGelu) {
    if (tiny) decode::fused_int4_kernel<kActGelu, true><<<g, b, 0, s>>>(p, q);
    else decode::fused_int4_kernel<kActGelu, false><<<g, b, 0, s>>>(p, q);
  } else {
    if (tiny) decode::fused_int4_kernel<kActSilu, true><<<g, b, 0, s>>>(p, q);
    else decode::fused_int4_kernel<kActSilu, false><<<g, b, 0, s>>>(p, q);
  }
  return fmoe_host::check_launch("fused_int4");
}

int launch_decode(WType wt, Mode mode, const GemmParams& p0, hipStream_t s) {
  GemmParams p = p0;
  const int64_t ncols = mode == Mode::kGemm1Silu ? p.N_act : p.Nout;
  const int per_block = mode == Mode::kGemm1Silu ? decode::BN / 2 : decode::BN;
  const int rbk = decode_row_blocks(wt);
  const int64_t nblocks = (ncols + per_block - 1) / per_block;
  p.n_ntiles = static_cast<int>((nblocks + rbk - 1) / rbk);  // workgroups along the output rows
  if (p.max_tiles <= 0) return FMOE_OK;
  dim3 g(static_cast<unsigned>(p.max_tiles), static_cast<unsigned>(p.n_ntiles),
         static_cast<unsigned>(mode == Mode::kGemm2 ? p.splits : 1));
  if (wt == WType::kInt4 && !p.tiny_ids && decode_int4_row_split(p.max_tiles) > 0) {
    g.y = static_cast<unsigned>((nblocks + decode::kRsBlocks - 1) / decode::kRsBlocks);
    const dim3 b(decode::kRsThreads);
    if (decode_int4_pair(p.max_tiles, p.n_experts)) {
      if (mode == Mode::kGemm2)
        decode::gemm_decode_int4_rs_kernel<Mode::kGemm2, kActSilu, true><<<g, b, 0, s>>>(p);
      else if (p.act == kActSwiglu)
        decode::gemm_decode_int4_rs_kernel<Mode::kGemm1Silu, kActSwiglu, true><<<g, b, 0, s>>>(p);
      else if (p.act == kActGelu)
        decode::gemm_decode_int4_rs_kernel<Mode::kGemm1Silu, kActGelu, true><<<g, b, 0, s>>>(p);
      else
        decode::gemm_decode_int4_rs_kernel<Mode::kGemm1Silu, kActSilu, true><<<g, b, 0, s>>>(p);
    } else {
      if (mode == Mode::kGemm2)
        decode::gemm_decode_int4_rs_kernel<Mode::kGemm2, kActSilu, false><<<g, b, 0, s>>>(p);
      else if (p.act == kActSwiglu)
        decode::gemm_decode_int4_rs_kernel<Mode::kGemm1Silu, kActSwiglu, false><<<g, b, 0, s>>>(p);
      else if (p.act == kActGelu)
        decode::gemm_decode_int4_rs_kernel<Mode::kGemm1Silu, kActGelu, false><<<g, b, 0, s>>>(p);
      else
        decode::gemm_decode_int4_rs_kernel<Mode::kGemm1Silu, kActSilu, false><<<g, b, 0, s>>>(p);
    }
    return fmoe_host::check_launch("gemm_decode_int4_rs");
  }
#define LAUNCH(WT_, MODE_, ACT_)                                                                      \
  do {                                                                                                \
    constexpr int RB_ = decode_row_blocks(WT_);                                                       \
    const dim3 b_(decode::kThreads * RB_);                                                            \
    if (p.tiny_ids && WT_ != WType::kMxfp4)                                                          \
      decode::gemm_decode_kernel<WT_, MODE_, decode::pipe_depth(WT_, MODE_, true), ACT_, true, RB_><<<g, b_, 0, s>>>(p); \
    else                                                                                              \
      decode::gemm_decode_kernel<WT_, MODE_, decode::pipe_depth(WT_, MODE_, false), ACT_, false, RB_><<<g, b_, 0, s>>>(p); \
  } while (0)
#define LAUNCH_G1(WT_)                                    \
  do {                                                    \
    if (p.act == kActSwiglu) LAUNCH(WT_, Mode::kGemm1Silu, kActSwiglu); \
    else if (p.act == kActGelu) LAUNCH(WT_, Mode::kGemm1Silu, kActGelu); \
    else LAUNCH(WT_, Mode::kGemm1Silu, kActSilu);        \
  } while (0)
  if (mode == Mode::kGemm1Silu) {
    switch (wt) {
      case WType::kBf16: LAUNCH_G1(WType::kBf16); break;
      case WType::kFp8: LAUNCH_G1(WType::kFp8); break;
      case WType::kInt4: LAUNCH_G1(WType::kInt4); break;
      case WType::kMxfp4: LAUNCH_G1(WType::kMxfp4); break;
    }
  } else {
    switch (wt) {
      case WType::kBf16: LAUNCH(WType::kBf16, Mode::kGemm2, kActSilu); break;
      case WType::kFp8: LAUNCH(WType::kFp8, Mode::kGemm2, kActSilu); break;
      case WType::kInt4: LAUNCH(WType::kInt4, Mode::kGemm2, kActSilu); break;
      case WType::kMxfp4: LAUNCH(WType::kMxfp4, Mode::kGemm2, kActSilu); break;
    }
  }
#undef LAUNCH_G1
#undef LAUNCH
  return fmoe_host::check_launch("gemm_decode");
}

// ---- small bf16 decode batches (M * k <= 32 slots): GEMM2 and the top-k sum
// in one launch.  out[t][r] = bf16(scale * sum_j g_tj * (w2[e_tj][r] . act_tj
// + b2[e_tj][r])), each token's slots j in ascending order (dropped ids
// skipped), as fmoe_moe_sum adds the per-slot rows of the two-launch path.  A
// workgroup owns one output row, so the grid (K rows) spreads evenly over the
// CUs; its 16 groups of 16 lanes take the (slot, reduction slice) items, S =
// ceil(16 / slots) slices so that few slots still fill the groups; each lane
// dots 8 columns per 16-byte load, 4 loads in flight; a group reduces with
// xor shuffles and the item sums meet in LDS, added in fixed (slot, slice)
// order: every run gives the same bits.
namespace decode {
constexpr int kTokSlots = 32;
template <int ROWS>
__global__ __launch_bounds__(256) void gemm2_sum_token_kernel(GemmParams q, int E, int k, float scale,
                                                              uint16_t* __restrict__ out) {
  constexpr int kGroups = 256 / 16;
  __shared__ float part[ROWS * kTokSlots];  // [(rr * slots + slot) * S + s]: items <= ROWS * 32
  const int grp = threadIdx.x / 16, sub = threadIdx.x % 16;
  const int64_t K = q.Nout, N = q.Kred;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * ROWS;
  const int slots = static_cast<int>(q.n_tokens) * k;
  const int S = ROWS * slots >= kGroups ? 1 : (kGroups + ROWS * slots - 1) / (ROWS * slots);
  const int64_t slice = ((N / 8 + S - 1) / S) * 8;
  const uint16_t* __restrict__ w2 = reinterpret_cast<const uint16_t*>(q.B);
  const uint16_t* __restrict__ act = reinterpret_cast<const uint16_t*>(q.A);
  for (int it = grp; it < ROWS * slots * S; it += kGroups) {
    const int rs = it / S, sl = it - (it / S) * S;
    const int rr = rs / slots, f = rs - (rs / slots) * slots;  // row in the block, flat slot t * k + j
    const int64_t row = row0 + rr;
    const int e = q.tiny_ids[f];
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (e >= 0 && e < E && row < K) {
      const uint16_t* wr = w2 + (static_cast<int64_t>(e) * K + row) * N;
      const uint16_t* ar = act + static_cast<int64_t>(f) * N;
      const int64_t n1 = min(N, (sl + 1) * slice);
      for (int64_t n = sl * slice + sub * 8; n < n1; n += 4 * 128) {
        i32x4_t w[4], a[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t c = n + u * 128 < n1 ? n + u * 128 : n;  // past the end: reread, not added
          w[u] = *reinterpret_cast<const i32x4_t*>(wr + c);
          a[u] = *reinterpret_cast<const i32x4_t*>(ar + c);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (n + u * 128 >= n1) continue;
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const uint32_t wv = static_cast<uint32_t>(w[u][h]), av = static_cast<uint32_t>(a[u][h]);
            acc[u] = __builtin_fmaf(__uint_as_float(wv << 16), __uint_as_float(av << 16), acc[u]);
            acc[u] = __builtin_fmaf(__uint_as_float(wv & 0xffff0000u), __uint_as_float(av & 0xffff0000u), acc[u]);
          }
        }
      }
    }
    float v = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    if (sub == 0) part[it] = v;
  }
  __syncthreads();
  const int rr = threadIdx.x / kTokSlots, t = threadIdx.x % kTokSlots;  // 256 / 32 = 8 >= ROWS
  const int64_t row = row0 + rr;
  if (rr < ROWS && t < q.n_tokens && row < K) {
    float y = 0.f;
    for (int j = 0; j < k; ++j) {
      const int f = t * k + j;
      const int e = q.tiny_ids[f];
      if (e < 0 || e >= E) continue;
      float d = 0.f;
      for (int sl = 0; sl < S; ++sl) d += part[(rr * slots + f) * S + sl];
      if (q.bias) d += q.bias[static_cast<int64_t>(e) * K + row];
      y += d * (q.gamma ? q.tiny_w[f] : 1.0f);
    }
    out[static_cast<int64_t>(t) * K + row] = f32_to_bf16(y * scale);
  }
}
}  // namespace decode

// ---- single-token bf16 decode GEMM1: act[j][c] = act(w13[e_j] rows of column
// c . x), one workgroup per (slot j, 8 columns): its 16 groups of 16 lanes
// each dot one weight row (the gate or up row of a column) with the token's
// x, 16-byte loads, 4 in flight; the epilogue is the row-block kernel's
// (gemm1_bias / gemm1_act, bf16 activation row).  Small N_act has more
// workgroups here than 64-row blocks give (Qwen3: 768 instead of 192).
namespace decode {
constexpr int kTokCols = 8;
template <int ACT>
__global__ __launch_bounds__(256) void gemm1_token_kernel(GemmParams p, int E) {
  __shared__ float dots[2 * kTokCols];
  const int grp = threadIdx.x / 16, sub = threadIdx.x % 16;
  const int64_t nblk = (p.N_act + kTokCols - 1) / kTokCols;
  const int j = static_cast<int>(blockIdx.x / nblk);
  const int64_t c0 = (blockIdx.x - static_cast<int64_t>(j) * nblk) * kTokCols;
  const int e = p.tiny_ids[j];
  if (e < 0 || e >= E) return;  // dropped slot: GEMM2 skips it
  const int64_t K = p.Kred;
  const int64_t col = c0 + grp / 2;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (col < p.N_act) {
    const uint16_t* wr = reinterpret_cast<const uint16_t*>(p.B) +
                         (static_cast<int64_t>(e) * p.Nout + gemm1_row(ACT, p.N_act, col, grp % 2)) * K;
    const uint16_t* xr = reinterpret_cast<const uint16_t*>(p.A);
    for (int64_t n = sub * 8; n < K; n += 4 * 128) {
      i32x4_t w[4], a[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t c = n + u * 128 < K ? n + u * 128 : n;  // past the end: reread, not added
        w[u] = *reinterpret_cast<const i32x4_t*>(wr + c);
        a[u] = *reinterpret_cast<const i32x4_t*>(xr + c);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (n + u * 128 >= K) continue;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint32_t wv = static_cast<uint32_t>(w[u][h]), av = static_cast<uint32_t>(a[u][h]);
          acc[u] = __builtin_fmaf(__uint_as_float(wv << 16), __uint_as_float(av << 16), acc[u]);
          acc[u] = __builtin_fmaf(__uint_as_float(wv & 0xffff0000u), __uint_as_float(av & 0xffff0000u), acc[u]);
        }
      }
    }
  }
  float v = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  if (sub == 0) dots[grp] = v;
  __syncthreads();
  const int t = threadIdx.x;
  if (t < kTokCols && c0 + t < p.N_act) {
    const float g = p.gamma ? p.tiny_w[j] : 1.0f;
    float gb, ub;
    gemm1_bias<ACT>(p, e, c0 + t, gb, ub);
    uint16_t* act = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(j) * p.N_act;
    act[c0 + t] = f32_to_bf16(gemm1_act<ACT>(p, dots[2 * t], dots[2 * t + 1], gb, ub, g));
  }
}
}  // namespace decode

// Single-token bf16 GEMM1 (p as for the row-block kernel with tiny routing).
int launch_gemm1_token(const GemmParams& p, int E, int k, hipStream_t s) {
  if (p.n_tokens != 1 || k < 1 || p.Kred % 8 != 0)
    return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "gemm1_token: one token, K %% 8 == 0");
  const int64_t grid = static_cast<int64_t>(k) * ((p.N_act + decode::kTokCols - 1) / decode::kTokCols);
  if (grid > 0x7fffffff) return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "gemm1_token: grid too large");
  const dim3 g(static_cast<unsigned>(grid)), b(256);
  if (p.act == kActSwiglu) decode::gemm1_token_kernel<kActSwiglu><<<g, b, 0, s>>>(p, E);
  else if (p.act == kActGelu) decode::gemm1_token_kernel<kActGelu><<<g, b, 0, s>>>(p, E);
  else decode::gemm1_token_kernel<kActSilu><<<g, b, 0, s>>>(p, E);
  return fmoe_host::check_launch("gemm1_token");
}

// Small-batch bf16 GEMM2 + top-k sum (q as for the two-launch path: A = the
// GEMM1 rows of the batch's flat slots, B = w2, tiny_ids / tiny_w / n_tokens
// the routing).
int launch_gemm2_sum_token(const GemmParams& q, int E, int k, float scale, void* out, hipStream_t s) {
  if (k < 1 || q.n_tokens < 1 || q.n_tokens * k > decode::kTokSlots || q.Kred % 8 != 0 || q.Nout < 1)
    return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "gemm2_sum_token: M * k <= %d, N %% 8 == 0",
                           decode::kTokSlots);
  if (q.Nout > 0x7fffffff) return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "gemm2_sum_token: K too large");
  // 4 output rows per workgroup while that still leaves >= 512 workgroups
  // (fewer, larger workgroups for short rows), else one row per workgroup
  if (q.Nout >= 2048 && q.Nout % 4 == 0)
    decode::gemm2_sum_token_kernel<4><<<dim3(static_cast<unsigned>(q.Nout / 4)), dim3(256), 0, s>>>(
        q, E, k, scale, static_cast<uint16_t*>(out));
  else
    decode::gemm2_sum_token_kernel<1><<<dim3(static_cast<unsigned>(q.Nout)), dim3(256), 0, s>>>(
        q, E, k, scale, static_cast<uint16_t*>(out));
  return fmoe_host::check_launch("gemm2_sum_token");
}

}  // namespace fmoe
