// Prefill grouped GEMM: one expert per M-tile; MFMA tiles fed from a ring of
// LDS stages filled by direct-to-LDS DMA.
//
// Workgroup = 8 waves (512 threads) laid out WAVES_M x WAVES_N; tile BM x BN;
// SB bytes of the reduction dim per row per stage (bf16: SB = 64 or 128 ->
// one or two v_mfma_f32_16x16x32_bf16 steps; fp8: SB = 128 -> one 128-wide
// scale block, one v_mfma_f32_16x16x128_f8f6f4 with its result scaled by
// a_scale[row] * w_scale[block] into the fp32 accumulator).
//
// Measured on MI355X, which is what the structure follows:
//  * DMA: global_load_lds_dwordx4 delivers ~2x the bytes per clock when
//    consecutive lanes read one row's contiguous bytes (4 or 8 lanes x 16 B)
//    than when every lane reads a different row.  LDS: a ds_read_b128
//    fragment read runs at full rate only if each 8 consecutive lanes hit 8
//    distinct 16-byte columns of a 128-byte window.  A stage is therefore a
//    set of 1 KiB units in row-major, XOR-swizzled layouts (see frag_off):
//    one unit is one wave-instruction of DMA, written without staging
//    registers or ds_write, and every fragment read is conflict-free.
//  * With the DMA running, operand delivery (not LDS or MFMA issue) bounds
//    the kernel, so the tile is as large as LDS allows (256 x 256 for bf16:
//    128 flop per byte moved) and two or three stages are kept in flight.
// Lane group g = L/16 sees reduction bytes 16g..16g+15 of each 64-byte half in
// both operands, so the MFMA dot products are exact permutations of the
// textbook ones.
//
// The DMA is issued from inline asm (M0 = LDS destination): the compiler then
// does not treat the LDS ring as written by an outstanding vector-memory op
// (it would insert vmcnt(0) before every fragment read).  Completion is
// ordered explicitly: per-wave vmcnt wait for the stage, then s_barrier
// without a fence (later stages keep streaming across it).
//
// GEMM1 (gate/up + SiLU): each wave's BN/WAVES_N weight rows are half gate rows
// and the matching up rows, so gate block j and up block j sit in the same
// lanes; silu(gate) * up is formed in registers and only the bf16 activation
// is written.  GEMM2: rows scaled by the routing weight; each slot row is
// stored as bf16 (one split), as fp32 split-K planes (stage-level calls), or,
// for the tail tiles of the fused path's tail split, as fp32 parts that
// tail_fold_kernel adds; the top-k sum runs in its own fixed-order launch
// (deterministic).
#include <algorithm>

#include "gemm.hpp"

namespace fmoe {
namespace prefill {

constexpr int kUnit = 1024;       // one DMA wave-instruction: 64 lanes x 16 B
constexpr int kMaxKStages = 128;  // fp8: reduction dims up to 16384 (64 stages when LDS is short)
constexpr int kGroupTiles = 32;   // tiles per rasterization window (~ one XCD's CUs)

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int SB_, int NBUF_, bool FP8_, Mode MODE_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WAVES_M = WAVES_M_, WAVES_N = WAVES_N_, SB = SB_,
                       NBUF = NBUF_;
  static constexpr bool FP8 = FP8_;
  static constexpr Mode MODE = MODE_;
  static constexpr int NW = WAVES_M * WAVES_N, NT = NW * 64;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int MI = WM / 16, NI = WN / 16;
  static constexpr int UPB = SB / 64;                       // units per 16-row block
  static_assert(SB == 64 || SB == 128, "stage width");
  static constexpr int A_UNITS = (BM / 16) * UPB, B_UNITS = (BN / 16) * UPB;
  // unit u of a stage is DMAed by wave u % NW: waves below REM (or all of
  // them when REM == 0) issue UPW units per stage, the others UPW - 1
  static constexpr int UNITS = A_UNITS + B_UNITS;
  static constexpr int UPW = (UNITS + NW - 1) / NW;
  static constexpr int REM = UNITS % NW;
  static constexpr int STAGE = UNITS * kUnit;
  // waves that DMA the activation scales (64 rows each): the last SA_WAVES
  // waves, which carry the fewer units when the split is uneven
  static constexpr int SA_WAVES = FP8 ? (BM + 63) / 64 : 0;
  static constexpr int SA_FIRST = NW - SA_WAVES;
  // fp8 weight-scale stages held in LDS (the reduction dim is at most 128 KST)
  static constexpr int KST =
      NBUF * STAGE + NBUF * BM * 4 + WAVES_N * 2 * kMaxKStages * 4 <= 160 * 1024 ? kMaxKStages : 64;
  static_assert(BM % 16 == 0 && (A_UNITS % 2) == 0, "16-row blocks");
  static_assert(REM == 0 || REM <= SA_FIRST || !FP8, "a-scale waves carry the fewer units");
  static_assert(!FP8 || SB == 128, "fp8 stages hold one 128-wide scale block");
  static_assert(MODE != Mode::kGemm1Silu || NI % 2 == 0, "gate/up pairing needs even NI");
  static_assert(NBUF >= 2 && NBUF <= 4, "ring depth");
  static_assert(NBUF * STAGE + NBUF * BM * 4 + WAVES_N * 2 * KST * 4 <= 160 * 1024, "LDS budget");
  static_assert(SA_WAVES <= NW, "a-scale waves");
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// wait until at most `newer` stages (P loads each) of this wave are in flight
template <int P>
__device__ __forceinline__ void wait_ring(int newer) {
  if (newer >= 2) wait_vmcnt<2 * P>();
  else if (newer == 1) wait_vmcnt<P>();
  else wait_vmcnt<0>();
}

__device__ __forceinline__ void barrier_nofence() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void* l) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)(l)));
}
// lane i's 16 (or 4) bytes land at LDS address l + 16 i (4 i)
__device__ __forceinline__ void dma16(const uint8_t* g, uint8_t* l) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr(l));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const float* g, float* l) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr(l));
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(g), "s"(m0) : "memory", "m0");
}

// LDS unit layouts (1 KiB = one DMA wave-instruction, lane i -> bytes 16i):
//  * 64-byte stages: a unit is 16 rows x 64 bytes; DMA lane i reads row i / 4,
//    chunk (i % 4) ^ ((row / 2) % 4), so 4 consecutive lanes read one row's 64
//    contiguous bytes.
//  * 128-byte stages: a unit is 8 rows x 128 bytes (rows 0-7 or 8-15 of a
//    16-row block); DMA lane i reads row i / 8, chunk (i % 8) ^ (row), so 8
//    consecutive lanes read one row's 128 contiguous bytes.
// The MFMA fragment of lane L is row L % 16, 16-byte chunk c (c = L / 16, and
// for 128-byte stages also 4 + L / 16); with the swizzles above every 8
// consecutive lanes of a fragment read hit 8 distinct 16-byte columns of a
// 128-byte window, which ds_read_b128 serves at the contiguous rate
// (measured: plain row-major or a (row / 4) swizzle run at 70% of it).
template <int SB>
__device__ __forceinline__ int frag_off(int L, int c) {
  const int r = L & 15;
  if constexpr (SB == 64) return 16 * (4 * r + (c ^ ((r >> 1) & 3)));
  const int ru = r & 7;
  return (r >> 3) * 1024 + 16 * (8 * ru + (c ^ ru));
}

__device__ __forceinline__ i32x4_t lds16(const uint8_t* p) { return *reinterpret_cast<const i32x4_t*>(p); }

// Expert e with offs_pad[e] * nn <= key < offs_pad[e + 1] * nn (offs_pad is
// non-decreasing, offs_pad[0] = 0, key < offs_pad[E] * nn): two rounds of 64
// parallel probes and a ballot, instead of a serial binary search.
__device__ __forceinline__ int find_expert(const int32_t* offs_pad, int E, int key, int nn, int lane) {
  const int S = (E + 1 + kWave - 1) / kWave;
  const int i1 = min(lane * S, E);
  uint64_t b = __ballot(offs_pad[i1] * nn <= key);
  const int base = (63 - __builtin_clzll(b)) * S;
  const int i2 = min(base + lane, E);
  b = __ballot(lane < S && offs_pad[i2] * nn <= key);
  return base + (63 - __builtin_clzll(b));
}

// 4x4 transpose across each quad of lanes (q = lane % 4): on entry v[r] of
// lane q is element (column q, row r), on exit v[c] is element (column c,
// row q).  Two exchange steps (lane bit 0 with element bit 0, then bit 1),
// each two DPP quad permutes.
template <int CTRL>
__device__ __forceinline__ float qperm(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ void quad_transpose(f32x4_t& v, int lane) {
  const bool p0 = lane & 1, p1 = lane & 2;
  float s0 = p0 ? v[0] : v[1], s1 = p0 ? v[2] : v[3];
  float r0 = qperm<0xB1>(s0), r1 = qperm<0xB1>(s1);  // quad_perm [1,0,3,2]
  if (p0) {
    v[0] = r0;
    v[2] = r1;
  } else {
    v[1] = r0;
    v[3] = r1;
  }
  s0 = p1 ? v[0] : v[2];
  s1 = p1 ? v[1] : v[3];
  r0 = qperm<0x4E>(s0);  // quad_perm [2,3,0,1]
  r1 = qperm<0x4E>(s1);
  if (p1) {
    v[0] = r0;
    v[1] = r1;
  } else {
    v[2] = r0;
    v[3] = r1;
  }
}

// Logical tile L (within one split) -> expert, N-tile and rows.  Per expert,
// windows of all its T M-tiles x G N-tiles (T * G ~ group_tiles, about what
// one XCD runs at once) are enumerated M-fastest, so the tiles that share a
// weight panel run together on one XCD and the panel is fetched from HBM
// once.  Called by one whole wave (find_expert ballots).
struct Tile {
  int e, nt, row_beg, row_end;
};
template <int BM>
__device__ __forceinline__ Tile tile_of(const GemmParams& p, int L, int lane) {
  const int nn = p.n_ntiles;
  Tile t;
  t.e = find_expert(p.offs_pad, p.n_experts, L, nn, lane);
  const int t0 = p.offs_pad[t.e];
  const int T = p.offs_pad[t.e + 1] - t0;
  const int local = L - t0 * nn;
  const int G = max(1, p.group_tiles / T);
  const int grp = local / (T * G);
  const int rr = local - grp * T * G;
  const int blk = rr % T;
  t.nt = grp * G + rr / T;
  t.row_beg = p.offs_raw[t.e] + blk * BM;
  t.row_end = min(p.offs_raw[t.e + 1], t.row_beg + BM);
  return t;
}

// Tail split of XCD x (GEMM2, p.tail_split > 1): the XCD's logical tiles are
// [base, base + Tx) (xcd_remap's partition of the T live tiles).  Whole
// tiles fill rounds of `slots` workgroups; the tl = Tx % slots tiles of the
// last partial round are split S = min(max_split, slots / tl, stages) ways,
// so their tl * S workgroups fill at most one round.  S = 1: no split, every
// tile whole.  The GEMM and tail_fold_kernel derive the same plan.
struct TailPlan {
  int base, full, tl, S;
};
__device__ __forceinline__ TailPlan tail_plan(int T, int x, int max_split, int slots, int stages) {
  const int q = T / kNumXcd, r8 = T % kNumXcd;
  const int Tx = q + (x < r8 ? 1 : 0);
  TailPlan t;
  t.base = x * q + min(x, r8);
  t.tl = Tx % slots;
  t.S = t.tl > 0 ? min(min(max_split, slots / t.tl), stages) : 1;
  if (t.S < 2) {
    t.S = 1;
    t.tl = 0;
  }
  t.full = Tx - t.tl;
  return t;
}
// Index of XCD x's first tail pair: the pairs of XCDs 0 .. x-1 come first.
__device__ __forceinline__ int tail_offset(int T, int x, int max_split, int slots, int stages) {
  int off = 0;
  for (int y = 0; y < x; ++y) {
    const TailPlan t = tail_plan(T, y, max_split, slots, stages);
    off += t.tl * t.S;
  }
  return off;
}

// Fills p.tile_lut for every live logical tile: one wave per tile.
template <int BM>
__global__ __launch_bounds__(256) void tile_lut_kernel(GemmParams p) {
  const int lane = threadIdx.x % kWave;
  const int L = blockIdx.x * 4 + threadIdx.x / kWave;
  if (L >= *p.n_tiles * p.n_ntiles) return;
  const Tile t = tile_of<BM>(p, L, lane);
  if (lane == 0) p.tile_lut[L] = int4{t.e, t.nt, t.row_beg, t.row_end};
}

// Adds the tail-split partials of each split tile in split order and writes
// the tile's bf16 rows (y_bf16 layout [slot][Nout]): one workgroup per (XCD,
// tail tile, 16-row chunk), every partial of the chunk loaded before the
// adds.  Bias and routing weight are already in the partials.
constexpr int kFoldRows = 16;
template <int BM, int BN>
__global__ __launch_bounds__(256) void tail_fold_kernel(GemmParams p, int stages) {
  constexpr int kChunks = BM / kFoldRows;
  constexpr int kVec = kFoldRows * BN / (4 * 256);  // float4 per thread and partial
  static_assert(kFoldRows * BN % (4 * 256) == 0, "fold chunk");
  const int rc = blockIdx.x % kChunks;
  const int xt = blockIdx.x / kChunks;
  const int x = xt / p.tail_slots, t = xt % p.tail_slots;
  const int T = *p.n_tiles * p.n_ntiles;
  const TailPlan pl = tail_plan(T, x, p.tail_split, p.tail_slots, stages);
  if (t >= pl.tl) return;
  const int pair0 = tail_offset(T, x, p.tail_split, p.tail_slots, stages) + t * pl.S;
  if (pair0 + pl.S > p.tail_pairs) return;
  const int L = pl.base + pl.full + t;
  int nt, rb, re;
  if (p.tile_lut) {
    const int4 v = p.tile_lut[L];
    nt = v.y;
    rb = v.z;
    re = v.w;
  } else {
    const Tile tt = tile_of<BM>(p, L, threadIdx.x % kWave);
    nt = tt.nt;
    rb = tt.row_beg;
    re = tt.row_end;
  }
  const int r0 = rc * kFoldRows;
  if (r0 >= re - rb) return;
  const int64_t c0 = static_cast<int64_t>(nt) * BN;
  const int cols = static_cast<int>(min(static_cast<int64_t>(BN), p.Nout - c0));
  const float* part = p.tail_part + static_cast<int64_t>(pair0) * (BM * BN) + r0 * BN;
  float4 a[kVec];
#pragma unroll
  for (int v = 0; v < kVec; ++v) a[v] = *reinterpret_cast<const float4*>(part + (threadIdx.x + v * 256) * 4);
  for (int sp = 1; sp < pl.S; ++sp) {
    float4 b[kVec];
#pragma unroll
    for (int v = 0; v < kVec; ++v)
      b[v] = *reinterpret_cast<const float4*>(part + static_cast<int64_t>(sp) * (BM * BN) + (threadIdx.x + v * 256) * 4);
#pragma unroll
    for (int v = 0; v < kVec; ++v) {
      a[v].x += b[v].x;
      a[v].y += b[v].y;
      a[v].z += b[v].z;
      a[v].w += b[v].w;
    }
  }
  uint16_t* y = static_cast<uint16_t*>(p.out);
#pragma unroll
  for (int v = 0; v < kVec; ++v) {
    const int idx = (threadIdx.x + v * 256) * 4;
    const int r = idx / BN, c = idx - (idx / BN) * BN;
    if (r0 + r >= re - rb || c >= cols) continue;
    const uint32_t w0 = f32_to_bf16(a[v].x) | (static_cast<uint32_t>(f32_to_bf16(a[v].y)) << 16);
    const uint32_t w1 = f32_to_bf16(a[v].z) | (static_cast<uint32_t>(f32_to_bf16(a[v].w)) << 16);
    *reinterpret_cast<uint2*>(y + static_cast<int64_t>(rb + r0 + r) * p.Nout + c0 + c) = make_uint2(w0, w1);
  }
}

template <class C, int ACT>
__global__ __launch_bounds__(C::NT) void gemm_prefill_kernel(GemmParams p) {
  constexpr int BM = C::BM, BN = C::BN, WM = C::WM, WN = C::WN, MI = C::MI, NI = C::NI;
  constexpr int SB = C::SB, UPB = C::UPB, NW = C::NW, NBUF = C::NBUF;
  constexpr bool FP8 = C::FP8;
  constexpr Mode MODE = C::MODE;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NBUF][C::STAGE];
  __shared__ __attribute__((aligned(256))) float sa_lds[NBUF][FP8 ? BM : 1];
  __shared__ float sb_lds[C::WAVES_N][2][FP8 ? C::KST : 1];

  const int tid = threadIdx.x, lane = tid % kWave;
  const int wid = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wid / C::WAVES_N, wn = wid % C::WAVES_N;

  // ---- which (split, expert M-tile, N-tile): workgroup ids are made
  // XCD-contiguous, then mapped by tile_of (or its precomputed table).
  const int nn = p.n_ntiles;
  const int per_split = *p.n_tiles * nn;
  const int64_t kbytes = FP8 ? p.Kred : p.Kred * 2;  // bytes per operand row
  const int nk_all = static_cast<int>(kbytes / SB);
  int L, split, n_splits = p.splits;
  int tail = -1;  // tail-split workgroup: its pair index in p.tail_part
  if (MODE == Mode::kGemm2 && p.tail_split > 1) {
    const TailPlan t = tail_plan(per_split, static_cast<int>(blockIdx.x) % kNumXcd, p.tail_split,
                                 p.tail_slots, nk_all);
    const int i = static_cast<int>(blockIdx.x) / kNumXcd;  // dispatch position within the XCD
    if (i < t.full) {
      L = t.base + i;
      split = 0;
      n_splits = 1;
    } else {
      const int j = i - t.full;
      if (j >= t.tl * t.S) return;
      L = t.base + t.full + j / t.S;
      split = j % t.S;
      n_splits = t.S;
      tail = tail_offset(per_split, static_cast<int>(blockIdx.x) % kNumXcd, p.tail_split, p.tail_slots,
                         nk_all) + j;
      if (tail >= p.tail_pairs) return;  // the host sizes tail_part for every pair
    }
  } else {
    const int live = per_split * p.splits;
    if (static_cast<int>(blockIdx.x) >= live) return;
    L = xcd_remap(blockIdx.x, live);
    split = L / per_split;
    L -= split * per_split;
  }
  int e, nt, row_beg, row_end;
  if (p.tile_lut) {
    const int4 v = p.tile_lut[L];
    e = v.x;
    nt = v.y;
    row_beg = v.z;
    row_end = v.w;
  } else {
    const Tile t = tile_of<BM>(p, L, lane);
    e = t.e;
    nt = t.nt;
    row_beg = t.row_beg;
    row_end = t.row_end;
  }

  // GEMM2: waves whose rows are all padding skip their fragment reads and
  // MFMAs.  An expert's last M-tile is often nearly empty (Mixtral M=4096:
  // ~1024 +- 30 slots per expert, so about half the experts add a fifth
  // 256-row tile of a few dozen rows).  Measured: GEMM2 -0.5 to -1.5% on the
  // BASELINE prefill shapes; GEMM1 +2-3% with the same skip, so not there.
  const bool wave_live = C::WAVES_M == 1 || MODE == Mode::kGemm1Silu ||
                         __builtin_amdgcn_readfirstlane(row_end - row_beg > wm * WM);

  const int ksb = static_cast<int>(p.Kred / 128);      // fp8 scale blocks per row
  // split-K: this workgroup reduces stages [k0, k0 + nk)
  const int per_k = (nk_all + n_splits - 1) / n_splits;
  const int k0 = min(nk_all, split * per_k);
  const int nk = min(nk_all, k0 + per_k) - k0;

  auto a_src_row = [&](int r) -> int64_t {
    int s = row_beg + r;
    if (s >= row_end) s = row_beg;  // padding row: any valid row, result discarded
    return MODE == Mode::kGemm1Silu ? p.topk_indx[s] / p.top_k : s;
  };
  // ---- DMA sources: unit u = NW i + wid of the stage (A units first, then
  // B units) in the layout of frag_off.
  const uint8_t* Be = p.B + static_cast<int64_t>(e) * p.Nout * kbytes;
  const uint8_t* src[C::UPW];
  int loff[C::UPW];
  const bool full_wave = C::REM == 0 || wid < C::REM;  // issues UPW units (else UPW - 1)
#pragma unroll
  for (int i = 0; i < C::UPW; ++i) {
    const int u = min(NW * i + wid, C::UNITS - 1);
    const int b = u / UPB;
    int lr, coff;  // row within the 16-row block, byte offset in the row slice
    if constexpr (SB == 64) {
      lr = lane >> 2;
      coff = ((lane & 3) ^ ((lr >> 1) & 3)) * 16;
    } else {
      const int ru = lane >> 3;
      lr = (u % 2) * 8 + ru;
      coff = ((lane & 7) ^ ru) * 16;
    }
    loff[i] = u * kUnit;
    if (u < C::A_UNITS) {
      src[i] = p.A + a_src_row(b * 16 + lr) * kbytes + static_cast<int64_t>(k0) * SB + coff;
    } else {
      const int r = (b - BM / 16) * 16 + lr;  // row of the B tile
      int64_t brow;
      if (MODE == Mode::kGemm1Silu) {
        const int w = r / WN, within = r % WN;
        int64_t j = static_cast<int64_t>(nt) * (BN / 2) + w * (WN / 2) + (within % (WN / 2));
        if (j >= p.N_act) j = p.N_act - 1;  // past the last column (BN / 2 need not divide N)
        brow = gemm1_row(ACT, p.N_act, j, within < WN / 2 ? 0 : 1);
      } else {
        brow = static_cast<int64_t>(nt) * BN + r;
        if (brow >= p.Nout) brow = p.Nout - 1;
      }
      src[i] = Be + brow * kbytes + static_cast<int64_t>(k0) * SB + coff;
    }
  }
  // fp8: waves SA_FIRST + j DMA the activation scales of rows 64 j + lane
  // (lanes past BM stay idle)
  const int sa_j = wid - C::SA_FIRST;
  const bool sa_wave = FP8 && sa_j >= 0;
  const bool sa_lane = sa_wave && 64 * sa_j + lane < BM;
  const float* sa_src = nullptr;
  if (sa_wave) sa_src = p.a_scale + a_src_row(min(64 * sa_j + lane, BM - 1)) * ksb + k0;
  int sb_split = NI;  // GEMM2: 16-row blocks of the wave under its first weight-scale block
  auto issue = [&](int kt) {
    uint8_t* st = lds[kt % NBUF];
    const int64_t off = static_cast<int64_t>(kt) * SB;
#pragma unroll
    for (int i = 0; i < C::UPW; ++i)
      if (i + 1 < C::UPW || full_wave) dma16(src[i] + off, st + loff[i]);
    if (sa_wave) {
      if (64 * (sa_j + 1) <= BM) {
        dma4(sa_src + kt, &sa_lds[kt % NBUF][64 * sa_j]);
      } else if (sa_lane) {  // partial last 64-row group: masked lanes write nothing
        dma4(sa_src + kt, &sa_lds[kt % NBUF][64 * sa_j]);
      }
    }
  };

  f32x4_t acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // per-lane fragment offsets within a 16-row block's units
  const int foff0 = frag_off<SB>(lane, lane >> 4);
  const int foff1 = SB == 64 ? 0 : frag_off<SB>(lane, 4 + (lane >> 4));
  // The wave raises its issue priority for its fragment reads and MFMAs and
  // drops it before the next stage's wait and DMA issue: bf16 (Mixtral
  // M=4096 GEMM1 1.90 -> 1.86 ms, Qwen3 M=8192 GEMM1 -1%) and fp8 GEMM2
  // (DSV3 M=4096 -1.3%); fp8 GEMM1 keeps one level (+3.6% with it)
  constexpr int kPrio = (FP8 && MODE == Mode::kGemm1Silu) ? 0 : 1;
  auto compute = [&](int kt) {
    if (kPrio) __builtin_amdgcn_s_setprio(kPrio);
    const uint8_t* st = lds[kt % NBUF];
    const uint8_t* As = st + (wm * MI) * UPB * kUnit;
    const uint8_t* Bs = st + (C::A_UNITS + wn * NI * UPB) * kUnit;
    if constexpr (FP8) {
      i32x8_t fa[MI], fb[NI];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        i32x4_t lo = lds16(As + (2 * i) * kUnit + foff0), hi = lds16(As + (2 * i) * kUnit + foff1);
        fa[i] = i32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        i32x4_t lo = lds16(Bs + (2 * j) * kUnit + foff0), hi = lds16(Bs + (2 * j) * kUnit + foff1);
        fb[j] = i32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
      const float sb0 = sb_lds[wn][0][kt], sb1 = sb_lds[wn][1][kt];
      const float* sa_st = sa_lds[kt % NBUF];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        float sa[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sa[r] = sa_st[wm * WM + i * 16 + (lane >> 4) * 4 + r];
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          f32x4_t t = {0.f, 0.f, 0.f, 0.f};
          t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fa[i], fb[j], t, 0, 0, 0, 0, 0, 0);
          const float sb = (MODE == Mode::kGemm1Silu ? j >= NI / 2 : j >= sb_split) ? sb1 : sb0;
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] += t[r] * (sa[r] * sb);
        }
      }
    } else {
      // every fragment of the stage is read up front, the second k-step's
      // reads pinned between the first k-step's MFMAs (the scheduler would
      // otherwise issue them after those MFMAs to save registers): Mixtral
      // M=4096 GEMM1 1.95 -> 1.90 ms, GEMM2 1.06 -> 1.02 ms
      bf16x8_t fa[UPB][MI], fb[UPB][NI];
#pragma unroll
      for (int h = 0; h < UPB; ++h) {
        const int fo = h == 0 ? foff0 : foff1;
#pragma unroll
        for (int i = 0; i < MI; ++i)
          fa[h][i] = __builtin_bit_cast(bf16x8_t, lds16(As + i * UPB * kUnit + fo));
#pragma unroll
        for (int j = 0; j < NI; ++j)
          fb[h][j] = __builtin_bit_cast(bf16x8_t, lds16(Bs + j * UPB * kUnit + fo));
      }
#pragma unroll
      for (int h = 0; h < UPB; ++h)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NI; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[h][i], fb[h][j], acc[i][j], 0, 0, 0);
      if constexpr (UPB == 2) {
        // schedule: the first k-step's reads, then the second k-step's reads
        // spread over the first k-step's MFMAs, then the remaining MFMAs
        constexpr int NF = MI + NI;  // fragment reads per k-step
        __builtin_amdgcn_sched_group_barrier(0x100, NF, 0);
#pragma unroll
        for (int r = 0; r < NF; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * MI * NI - 2 * NF, 0);
      }
    }
    if (kPrio) __builtin_amdgcn_s_setprio(0);
  };

  // ring: up to NBUF-2 stages newer than kt stay in flight while kt is consumed
#pragma unroll
  for (int s = 0; s < NBUF - 1; ++s)
    if (s < nk) issue(s);
  // fp8 weight scales of the whole k range, staged once in LDS -- after the
  // first stages' DMA is issued, so the two round trips overlap
  if (FP8) {
    const int64_t nrb = p.Nout / 128;
    const float* se = p.b_scale + static_cast<int64_t>(e) * nrb * ksb;
    const float* s0;
    const float* s1;
    if (MODE == Mode::kGemm1Silu) {
      // the wave's gate rows (and up rows) lie in one 128-row scale block
      const int64_t j = static_cast<int64_t>(nt) * (BN / 2) + wn * (WN / 2);
      s0 = se + (gemm1_row(ACT, p.N_act, j, 0) / 128) * ksb;
      s1 = se + (gemm1_row(ACT, p.N_act, j, 1) / 128) * ksb;
    } else {
      // the wave's rows span at most two 128-row scale blocks (WN <= 128):
      // 16-row blocks j < sb_split use the first one
      int64_t j = static_cast<int64_t>(nt) * BN + wn * WN;
      if (j >= p.Nout) j = p.Nout - 1;
      const int64_t jl = min(j + WN - 1, p.Nout - 1);
      s0 = se + (j / 128) * ksb;
      s1 = se + (jl / 128) * ksb;
      if (jl / 128 != j / 128) sb_split = static_cast<int>((128 - j % 128) / 16);
    }
    if (wm == 0)
      for (int kk = lane; kk < nk; kk += kWave) {
        sb_lds[wn][0][kk] = s0[k0 + kk];
        sb_lds[wn][1][kk] = s1[k0 + kk];
      }
    __syncthreads();
  }

  // DMA instructions per stage for this wave: UPW or UPW - 1 operand units,
  // plus one a-scale load
  const int per = (full_wave ? C::UPW : C::UPW - 1) + (sa_wave ? 1 : 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int newer = min(NBUF - 2, nk - 1 - kt);
    if (per == C::UPW + 1) wait_ring<C::UPW + 1>(newer);
    else if (per == C::UPW) wait_ring<C::UPW>(newer);
    else wait_ring<(C::UPW > 1 ? C::UPW - 1 : 1)>(newer);
    barrier_nofence();
    if (kt + NBUF - 1 < nk) issue(kt + NBUF - 1);
    if (wave_live) compute(kt);
  }

  // ---- epilogue.  C layout of a 16x16 block: lane holds column lane%16,
  // rows 4*(lane/16) + r.  A 4x4 transpose inside each quad of lanes turns
  // that into row 4*(lane/16) + lane%4, columns 4*((lane/4)%4) + 0..3, so each
  // lane stores 4 consecutive outputs at once (8 or 16 bytes) instead of 4
  // scattered ones.
  const int orow = (lane >> 4) * 4 + (lane & 3);   // row within the 16x16 block
  const int ocol = ((lane >> 2) & 3) * 4;          // first of the lane's 4 columns
  // Routing weights of the lane's rows, loaded and waited for before the
  // first store.  On gfx9 loads and stores share the vmcnt counter and the
  // compiler treats them as completing out of order, so a use of a load that
  // is still pending after a store waits for every store before it
  // (vmcnt(0) at each of the tile's stores): the empty asm with the values as
  // operands makes the compiler complete the loads here, once.
  float gv[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int s = row_beg + wm * WM + i * 16 + orow;
    gv[i] = (p.gamma && s < row_end) ? p.gate_scal[s] : 1.0f;
  }
#pragma unroll
  for (int i = 0; i < MI; ++i) asm volatile("" ::"v"(gv[i]));
  // GEMM2 bias of the lane's columns (split 0 only), loaded the same way
  float bv[MODE == Mode::kGemm2 ? NI : 1][4] = {};
  if (MODE == Mode::kGemm2 && p.bias && split == 0) {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int64_t col = static_cast<int64_t>(nt) * BN + wn * WN + j * 16 + ocol;
      if (col < p.Nout) {
        const float* b = p.bias + static_cast<int64_t>(e) * p.Nout + col;
#pragma unroll
        for (int c = 0; c < 4; ++c) bv[j][c] = b[c];
      }
    }
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(bv[j][c]));
  }
  if constexpr (FP8 && MODE == Mode::kGemm1Silu && BN / 2 == 128) {
    if (p.act_q) {
      // Activation quantized here, exactly as fmoe_quant_fp8_group would do
      // it on the bf16 activation: the tile's 128 activation columns are one
      // 1x128 group of each row.  Row amax: the lane's 8 values, the 4 lanes
      // holding the row's other columns of this wave, then the WAVES_N waves
      // through LDS (the operand ring is free once every wave has left the
      // main loop).
      __syncthreads();
      float* amax_lds = reinterpret_cast<float*>(&lds[0][0]);  // [BM][WAVES_N]
      float v[MI][NI / 2][4];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const float g = gv[i];
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < NI / 2; ++j) {
          f32x4_t gv = acc[i][j], uv = acc[i][j + NI / 2];
          quad_transpose(gv, lane);
          quad_transpose(uv, lane);
          const int64_t col = static_cast<int64_t>(nt) * (BN / 2) + wn * (WN / 2) + j * 16 + ocol;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float gb, ub;
            gemm1_bias<ACT>(p, e, col + c, gb, ub);
            v[i][j][c] = round_bf16(gemm1_act<ACT>(p, gv[c], uv[c], gb, ub, g));
            amax = fmaxf(amax, fabsf(v[i][j][c]));
          }
        }
        amax = fmaxf(amax, __shfl_xor(amax, 4, kWave));
        amax = fmaxf(amax, __shfl_xor(amax, 8, kWave));
        if (((lane >> 2) & 3) == 0) amax_lds[(wm * WM + i * 16 + orow) * C::WAVES_N + wn] = amax;
      }
      __syncthreads();
      const int64_t ngrp = p.N_act / 128;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int r = wm * WM + i * 16 + orow;
        const int s = row_beg + r;
        float amax = 0.f;
#pragma unroll
        for (int w = 0; w < C::WAVES_N; ++w) amax = fmaxf(amax, amax_lds[r * C::WAVES_N + w]);
        const float sc = fmaxf(amax, kFp8Eps) / kFp8Max;
        const float inv = 1.0f / sc;
        if (s >= row_end) continue;
        uint8_t* q = p.act_q + static_cast<int64_t>(s) * p.N_act;
#pragma unroll
        for (int j = 0; j < NI / 2; ++j) {
          const int64_t col = static_cast<int64_t>(nt) * (BN / 2) + wn * (WN / 2) + j * 16 + ocol;
          *reinterpret_cast<uint32_t*>(q + col) =
              pack_e4m3x4(fp8_qdiv(v[i][j][0], sc, inv), fp8_qdiv(v[i][j][1], sc, inv),
                          fp8_qdiv(v[i][j][2], sc, inv), fp8_qdiv(v[i][j][3], sc, inv));
        }
        if (wn == 0 && ((lane >> 2) & 3) == 0) p.act_qs[static_cast<int64_t>(s) * ngrp + nt] = sc;
      }
      return;
    }
  }
  const bool y_rows_bf16 = p.y_bf16 && tail < 0;  // whole tile, one split: bf16 slot rows
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int s = row_beg + wm * WM + i * 16 + orow;
    const bool ok = s < row_end;
    const float g = gv[i];
    if (MODE == Mode::kGemm1Silu) {
      uint16_t* act = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(s) * p.N_act;
#pragma unroll
      for (int j = 0; j < NI / 2; ++j) {
        f32x4_t gv = acc[i][j], uv = acc[i][j + NI / 2];
        quad_transpose(gv, lane);
        quad_transpose(uv, lane);
        uint32_t w[2];
        const int64_t col = static_cast<int64_t>(nt) * (BN / 2) + wn * (WN / 2) + j * 16 + ocol;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          float a[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float gb, ub;
            gemm1_bias<ACT>(p, e, col + 2 * c + h, gb, ub);
            a[h] = gemm1_act<ACT>(p, gv[2 * c + h], uv[2 * c + h], gb, ub, g);
          }
          w[c] = f32_to_bf16(a[0]) | (static_cast<uint32_t>(f32_to_bf16(a[1])) << 16);
        }
        if (ok && col < p.N_act) *reinterpret_cast<uint2*>(act + col) = make_uint2(w[0], w[1]);
      }
    } else {
      // fp32 destination row: a split plane's slot row, or the tile's row of
      // its tail-split partial ([BM][BN] within the tile; the row pointer is
      // taken back by the tile's first column, which `col` adds again, so
      // both cases share one store)
      float* y = tail >= 0 ? p.tail_part + static_cast<int64_t>(tail) * (BM * BN) +
                                 (wm * WM + i * 16 + orow) * BN - static_cast<int64_t>(nt) * BN
                           : static_cast<float*>(p.out) + split * p.out_split_stride +
                                 static_cast<int64_t>(s) * p.Nout;
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        f32x4_t v = acc[i][j];
        quad_transpose(v, lane);
        const int64_t col = static_cast<int64_t>(nt) * BN + wn * WN + j * 16 + ocol;
        if (p.bias && split == 0) {
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] += bv[j][c];
        }
        if (ok && col < p.Nout) {
          if (y_rows_bf16) {
            // one split: the row goes out as bf16, like SGLang's per-slot
            // intermediate before its top-k sum
            uint16_t* yb = static_cast<uint16_t*>(p.out) + static_cast<int64_t>(s) * p.Nout + col;
            const uint32_t w0 = f32_to_bf16(v[0] * g) | (static_cast<uint32_t>(f32_to_bf16(v[1] * g)) << 16);
            const uint32_t w1 = f32_to_bf16(v[2] * g) | (static_cast<uint32_t>(f32_to_bf16(v[3] * g)) << 16);
            *reinterpret_cast<uint2*>(yb) = make_uint2(w0, w1);
          } else {
            *reinterpret_cast<float4*>(y + col) = make_float4(v[0] * g, v[1] * g, v[2] * g, v[3] * g);
          }
        }
      }
    }
  }
}

// Workgroup slots of one XCD for a configuration's kernel (workgroups per CU
// x CUs per XCD); 0 when the runtime cannot say (the tail split is then off).
template <class C>
int xcd_slots() {
  static const int slots = [] {
    int dev = 0, cus = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, gemm_prefill_kernel<C, kActSilu>, C::NT, 0) != hipSuccess) {
      (void)hipGetLastError();  // not left for the next launch's check to report
      return 0;
    }
    return (cus % kNumXcd == 0 && occ > 0) ? occ * (cus / kNumXcd) : 0;
  }();
  return slots;
}

// Partials the tail split of a GEMM2 launch may need: at most one round of
// an XCD's slots per XCD, and at most kTailMaxSplit per live tile.
template <class C>
int64_t tail_pairs_for(int64_t max_tiles, int64_t Nout) {
  const int slots = xcd_slots<C>();
  if (slots <= 0) return 0;
  const int64_t nn = (Nout + C::BN - 1) / C::BN;
  return std::min<int64_t>(static_cast<int64_t>(kNumXcd) * slots, max_tiles * nn * kTailMaxSplit);
}

template <class C>
int launch(const GemmParams& p0, hipStream_t s) {
  GemmParams p = p0;
  const int64_t ncols = C::MODE == Mode::kGemm1Silu ? p.N_act : p.Nout;
  const int per_tile = C::MODE == Mode::kGemm1Silu ? C::BN / 2 : C::BN;
  p.n_ntiles = static_cast<int>((ncols + per_tile - 1) / per_tile);
  if (p.group_tiles <= 0) p.group_tiles = kGroupTiles;
  if (p.splits < 1) p.splits = 1;
  int64_t grid = static_cast<int64_t>(p.max_tiles) * p.n_ntiles * p.splits;
  if (C::MODE == Mode::kGemm2 && p.tail_split > 1) {
    const int slots = xcd_slots<C>();
    const int64_t pairs = tail_pairs_for<C>(p.max_tiles, p.Nout);
    p.tail_pairs = static_cast<int64_t>(p.tail_bytes / (static_cast<size_t>(C::BM) * C::BN * sizeof(float)));
    if (slots <= 0 || !p.tail_part || pairs <= 0 || p.tail_pairs < pairs || p.splits != 1 || !p.y_bf16) {
      p.tail_split = 0;  // whole tiles only
    } else {
      p.tail_slots = slots;
      const int64_t per_xcd = (static_cast<int64_t>(p.max_tiles) * p.n_ntiles + kNumXcd - 1) / kNumXcd;
      grid = kNumXcd * (per_xcd + slots);  // whole tiles + one round of tail workgroups per XCD
    }
  }
  if (grid <= 0) return FMOE_OK;
  if (grid > 0x7fffffff) return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "prefill grid too large");
  if (C::FP8 && p.Kred / 128 > C::KST)
    return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "prefill fp8: reduction dim %lld is not supported",
                           static_cast<long long>(p.Kred));
  if (p.tile_lut) {
    const int64_t lut_n = static_cast<int64_t>(p.max_tiles) * p.n_ntiles;
    tile_lut_kernel<C::BM><<<dim3(static_cast<unsigned>((lut_n + 3) / 4)), dim3(256), 0, s>>>(p);
  }
  const dim3 g(static_cast<unsigned>(grid)), b(C::NT);
  if (C::MODE == Mode::kGemm2 || p.act == kActSilu)
    gemm_prefill_kernel<C, kActSilu><<<g, b, 0, s>>>(p);
  else if (p.act == kActGelu)
    gemm_prefill_kernel<C, kActGelu><<<g, b, 0, s>>>(p);
  else
    gemm_prefill_kernel<C, kActSwiglu><<<g, b, 0, s>>>(p);
  if (C::MODE == Mode::kGemm2 && p.tail_split > 1) {
    const int stages = static_cast<int>((C::FP8 ? p.Kred : 2 * p.Kred) / C::SB);
    tail_fold_kernel<C::BM, C::BN>
        <<<dim3(static_cast<unsigned>(kNumXcd * p.tail_slots * (C::BM / kFoldRows))), dim3(256), 0, s>>>(p, stages);
  }
  return fmoe_host::check_launch("gemm_prefill");
}

}  // namespace prefill

// Host launcher: picks the instantiation for the tile height.
//   bf16: BM 256 -> 256x256, 4x2 waves, 128-byte stages, 2-deep ring
//         BM 160 -> 160x256, 2x4 waves, 128-byte stages, 3-deep ring
//         BM 128 -> 128x256, 2x4 waves, 128-byte stages, 3-deep ring
//         BM  64 ->  64x256, 1x4 waves, 64-byte stages, 4-deep ring
//   fp8 : BM 160 -> GEMM1 160x256, 3-deep ring; GEMM2 160x384, 2-deep ring;
//                   2x4 waves, 128-byte stages (K, N <= 8192)
//         BM 128 -> 128x256, 2x4 waves, 128-byte stages, 3-deep ring
//         BM  64 ->  64x256, 1x8 waves, 128-byte stages, 3-deep ring
int launch_prefill(WType wt, Mode mode, int bm, const GemmParams& p, hipStream_t s) {
  using namespace prefill;
  const bool fp8 = wt == WType::kFp8;
#define L(BM, BN, WMS, WNS, SB, NB, F8)                                                      \
  (mode == Mode::kGemm1Silu ? launch<Cfg<BM, BN, WMS, WNS, SB, NB, F8, Mode::kGemm1Silu>>(p, s) \
                            : launch<Cfg<BM, BN, WMS, WNS, SB, NB, F8, Mode::kGemm2>>(p, s))
  if (!fp8) {
    if (bm == 256) return L(256, 256, 4, 2, 128, 2, false);
    if (bm == 160) return L(160, 256, 2, 4, 128, 3, false);
    if (bm == 128) return L(128, 256, 2, 4, 128, 3, false);
    if (bm == 64) return L(64, 256, 1, 4, 64, 4, false);
  } else {
    // GEMM2 with 160-row tiles: 384-wide output tiles (2-deep ring of 68 KiB
    // stages), so the activation tile is re-read by a third fewer N-tiles
    // (13% fewer operand requests per output; DSV3 GEMM2 M=4096 -5%, M=8192 -7%)
    if (bm == 160 && mode == Mode::kGemm2) return launch<Cfg<160, 384, 2, 4, 128, 2, true, Mode::kGemm2>>(p, s);
    if (bm == 160) return L(160, 256, 2, 4, 128, 3, true);
    if (bm == 128) return L(128, 256, 2, 4, 128, 3, true);
    if (bm == 64) return L(64, 256, 1, 8, 128, 3, true);
  }
#undef L
  return fmoe_host::fail(FMOE_ERR_UNSUPPORTED,
                         "prefill: block_m=%d is not supported for this weight type", bm);
}

// Bytes of the tail-split partial buffer for a fused prefill GEMM2 of this
// weight type and tile height (the configuration launch_prefill picks).
size_t prefill_tail_bytes(WType wt, int bm, int64_t max_tiles, int64_t Nout) {
  using namespace prefill;
#define T(BM, BN, WMS, WNS, SB, NB, F8) \
  static_cast<size_t>(tail_pairs_for<Cfg<BM, BN, WMS, WNS, SB, NB, F8, Mode::kGemm2>>(max_tiles, Nout)) * BM * BN * 4
  if (wt != WType::kFp8) {
    if (wt != WType::kBf16) return 0;
    if (bm == 256) return T(256, 256, 4, 2, 128, 2, false);
    if (bm == 160) return T(160, 256, 2, 4, 128, 3, false);
    if (bm == 128) return T(128, 256, 2, 4, 128, 3, false);
    if (bm == 64) return T(64, 256, 1, 4, 64, 4, false);
  } else {
    if (bm == 160) return T(160, 384, 2, 4, 128, 2, true);
    if (bm == 128) return T(128, 256, 2, 4, 128, 3, true);
    if (bm == 64) return T(64, 256, 1, 8, 128, 3, true);
  }
#undef T
  return 0;
}

}  // namespace fmoe
