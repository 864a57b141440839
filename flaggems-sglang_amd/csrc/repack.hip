// Load-time conversion of int4 MoE checkpoints (AWQ, GPTQ) into the layout the
// W4A16 kernels read.  Integer / byte work, HBM-bound, run once per weight.
//
// Source formats (per expert, stacked on a leading expert dim; K = reduction
// dim / input features, N = output rows / features, g = group size):
//   AWQ  (AutoAWQ "gemm" packing): qweight int32 [K, N/8]: word j of row k
//        holds columns 8j..8j+7, nibble i (bits 4i..4i+3) = column
//        8j + kAwqOrder[i]; qzeros int32 [K/g, N/8] packed the same way;
//        scales fp16 [K/g, N]; w = (q - z) * s.
//   GPTQ (AutoGPTQ packing, no act-order): qweight int32 [K/8, N]: word i of
//        column n holds rows 8i..8i+7, nibble j = row 8i + j; qzeros int32
//        [K/g, N/8], nibble j of word c = column 8c + j; scales fp16
//        [K/g, N].  Format v1 stores zero - 1 (w = (q - (z + 1)) * s), v2
//        stores the zero itself.
// Target (the W4A16 kernels): q u8 [N, K/2] (row n, reduction element 2i in
// the low nibble, 2i+1 in the high), scales fp16 [K/g, N] (unchanged), zeros
// u8 [K/g, N/2] (row 2j low nibble, 2j+1 high).
//
// GPTQ words are already packed along K in the target's nibble order, so their
// conversion is a transpose of 32-bit words; AWQ needs a 4-bit transpose,
// staged through LDS one 128 x 128 tile at a time.
#include "common.hpp"

namespace fmoe {
namespace repack {

constexpr int kTile = 64;    // GPTQ word-transpose tile
constexpr int kAwqTK = 128;  // AWQ nibble tile: reduction elements x output rows
constexpr int kAwqTN = 128;  // (measured best of 64/128/256 combinations)
constexpr int kThreads = 256;
// column held by nibble i of an AWQ word (within its 8 columns)
__constant__ int kAwqOrder[8] = {0, 2, 4, 6, 1, 3, 5, 7};
// nibble holding column c of an AWQ word (inverse of kAwqOrder)
__constant__ int kAwqNibble[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// AWQ qweight [E][K][N/8] -> q [E][N][K/2], one TK x TN tile (reduction x
// output rows) per workgroup through an LDS nibble tile.  Grid (N/TN, K/TK, E).
template <int TK, int TN>
__global__ __launch_bounds__(kThreads) void awq_weight_kernel(const int32_t* __restrict__ qw,
                                                              int64_t K, int64_t N,
                                                              uint8_t* __restrict__ out) {
  __shared__ uint8_t t[TN][TK + 4];  // [n][k]
  constexpr int WPR = TN / 8;         // words per tile row
  const int tid = threadIdx.x;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * TN;
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * TK;
  const int64_t e = blockIdx.z;
  const int64_t nw = N / 8;
  const int32_t* src = qw + e * K * nw;
  // consecutive threads read consecutive words of a row (TN / 2 bytes)
  for (int w = tid; w < TK * WPR; w += kThreads) {
    const int kl = w / WPR, jl = w % WPR;
    const int64_t k = k0 + kl, j = n0 / 8 + jl;
    uint32_t word = 0;
    if (k < K && j < nw) word = static_cast<uint32_t>(src[k * nw + j]);
#pragma unroll
    for (int i = 0; i < 8; ++i) t[8 * jl + kAwqOrder[i]][kl] = static_cast<uint8_t>((word >> (4 * i)) & 15u);
  }
  __syncthreads();
  // each thread writes 8 bytes (16 reduction elements) of one output row;
  // consecutive threads cover one row's TK / 2 bytes
  constexpr int PPR = TK / 16;  // 8-byte pieces per row
  for (int w = tid; w < TN * PPR; w += kThreads) {
    const int nl = w / PPR, part = w % PPR;
    const int64_t n = n0 + nl;
    if (n >= N) continue;
    uint8_t* dst = out + (e * N + n) * (K / 2);
    uint32_t b[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kl = 16 * part + 2 * i;
      const uint32_t byte = t[nl][kl] | (t[nl][kl + 1] << 4);
      b[i / 4] |= byte << (8 * (i % 4));
    }
    const int64_t kb = k0 + 16 * part;  // first reduction element of these 8 bytes
    if (kb + 16 <= K) {
      *reinterpret_cast<uint2*>(dst + kb / 2) = make_uint2(b[0], b[1]);
    } else {
      for (int i = 0; i < 8 && kb + 2 * i < K; ++i) dst[kb / 2 + i] = static_cast<uint8_t>(b[i / 4] >> (8 * (i % 4)));
    }
  }
}

// GPTQ qweight [E][K/8][N] -> q [E][N][K/2] viewed as words [E][N][K/8]: a
// 32-bit transpose.  Grid (N/64, K8/64, E), 256 threads.
__global__ __launch_bounds__(kThreads) void gptq_weight_kernel(const uint32_t* __restrict__ qw,
                                                               int64_t K8, int64_t N,
                                                               uint32_t* __restrict__ out) {
  __shared__ uint32_t t[kTile][kTile + 1];  // [i][n]
  const int tid = threadIdx.x;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int64_t i0 = static_cast<int64_t>(blockIdx.y) * kTile;
  const int64_t e = blockIdx.z;
  const uint32_t* src = qw + e * K8 * N;
  for (int w = tid; w < kTile * kTile; w += kThreads) {
    const int il = w / kTile, nl = w % kTile;  // consecutive threads: consecutive n
    const int64_t i = i0 + il, n = n0 + nl;
    t[il][nl] = (i < K8 && n < N) ? src[i * N + n] : 0u;
  }
  __syncthreads();
  uint32_t* dst = out + e * N * K8;
  for (int w = tid; w < kTile * kTile; w += kThreads) {
    const int nl = w / kTile, il = w % kTile;  // consecutive threads: consecutive i
    const int64_t i = i0 + il, n = n0 + nl;
    if (i < K8 && n < N) dst[n * K8 + i] = t[il][nl];
  }
}

// Zeros and scales: one thread per output zero byte (rows 2p, 2p+1 of group
// g of expert e).  `bad` counts GPTQ v1 zeros that overflow 4 bits.
__global__ __launch_bounds__(kThreads) void zeros_scales_kernel(int fmt, const uint32_t* __restrict__ qz,
                                                                const uint16_t* __restrict__ sc,
                                                                int64_t total_pairs, int64_t N,
                                                                uint8_t* __restrict__ zo,
                                                                uint16_t* __restrict__ so,
                                                                int32_t* __restrict__ bad) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= total_pairs) return;
  const int64_t half = N / 2;
  const int64_t row = idx / half;  // (e, g) flattened
  const int64_t p = idx % half;
  uint32_t z[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t c = 2 * p + h;
    const uint32_t word = qz[row * (N / 8) + c / 8];
    const int nib = fmt == FMOE_INT4_AWQ ? kAwqNibble[c % 8] : static_cast<int>(c % 8);
    uint32_t v = (word >> (4 * nib)) & 15u;
    if (fmt == FMOE_INT4_GPTQ_V1) {
      v += 1u;
      if (v > 15u && bad) atomicAdd(bad, 1);
      v &= 15u;
    }
    z[h] = v;
  }
  zo[idx] = static_cast<uint8_t>(z[0] | (z[1] << 4));
  so[row * N + 2 * p] = sc[row * N + 2 * p];
  so[row * N + 2 * p + 1] = sc[row * N + 2 * p + 1];
}

// FMOE_W_INT4 q [E][R][K/2] -> FMOE_W_INT4_TILED [E][R/16][K/128][1024]: one
// thread per 16-byte chunk, threads in source order (coalesced reads); chunk
// g of row 16b + r's 64-byte group slice c lands at 16 (16 g + r) of block
// (b, c).
__global__ __launch_bounds__(kThreads) void tile_int4_kernel(const i32x4_t* __restrict__ q,
                                                             int64_t chunks, int64_t K,
                                                             i32x4_t* __restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= chunks) return;
  const int64_t cpr = K / 32;  // 16-byte chunks per row (K/2 bytes)
  const int64_t row = idx / cpr;  // flattened over experts: e * R + r
  const int64_t ch = idx % cpr;
  const int64_t c = ch / 4, g = ch % 4;
  const int64_t b = row / 16, r = row % 16;
  out[(b * (K / 128) + c) * 64 + g * 16 + r] = q[idx];
}

// 4-bit weights -> bf16 [E][R][K] (the large-batch path runs the bf16 prefill
// kernels on them).  One thread per 8 elements of one row: a 4-byte source
// load and one 16-byte store, so a wave writes one contiguous KiB.  Source
// row-major [E][R][K/2] or tiled [E][R/16][K/128][1024] (fmoe_tile_int4).
//   int4 : w = (q - z) * s in fp32, rounded to bf16 (RNE);
//   MXFP4: w = e2m1(q) * 2^(s - 127), exact in bf16 (hardware conversion).
template <bool MX>
__global__ __launch_bounds__(kThreads) void dequant_4bit_kernel(const uint8_t* __restrict__ q,
                                                                int tiled, const void* __restrict__ scale,
                                                                const uint8_t* __restrict__ zeros,
                                                                int64_t units, int64_t R, int64_t K,
                                                                uint16_t* __restrict__ out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (idx >= units) return;
  const int64_t upr = K / 8;       // 8-element units per row
  const int64_t row = idx / upr;   // over all experts: e * R + r
  const int64_t m = idx % upr;     // elements 8m .. 8m+7 of the row
  const int64_t e = row / R, r = row % R;
  int64_t src;                     // byte offset of the unit's 4 source bytes
  if (tiled) {
    const int64_t c = m / 16, o = (m % 16) * 4;  // 128-element group, byte in its 64
    const int64_t rb = row / 16;                 // 16-row block over all experts
    src = (rb * (K / 128) + c) * 1024 + ((o / 16) * 16 + (row % 16)) * 16 + o % 16;
  } else {
    src = row * (K / 2) + 4 * m;
  }
  const uint32_t word = *reinterpret_cast<const uint32_t*>(q + src);
  uint32_t w[4];
  if constexpr (MX) {
    const uint8_t sb = static_cast<const uint8_t*>(scale)[row * (K / 32) + m / 4];
    const float sc = sb == 0 ? 0x1p-127f : (sb == 255 ? __builtin_nanf("") : __uint_as_float(static_cast<uint32_t>(sb) << 23));
    w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 0));
    w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 1));
    w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 2));
    w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, sc, 3));
  } else {
    const int64_t gbase = (e * (K / 128) + m / 16) * R;  // quant group m / 16 of expert e
    const float s = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(scale)[gbase + r]));
    const uint8_t zb = zeros[(gbase >> 1) + (r >> 1)];
    const float z = static_cast<float>((r & 1) ? (zb >> 4) : (zb & 15));
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float lo = (static_cast<float>((word >> (8 * b)) & 15u) - z) * s;
      const float hi = (static_cast<float>((word >> (8 * b + 4)) & 15u) - z) * s;
      w[b] = f32_to_bf16(lo) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
    }
  }
  *reinterpret_cast<i32x4_t*>(out + row * K + 8 * m) =
      i32x4_t{static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]), static_cast<int>(w[3])};
}

}  // namespace repack
}  // namespace fmoe

extern "C" int fmoe_repack_int4(int format, const int32_t* qweight, const int32_t* qzeros,
                                const uint16_t* scales, int64_t E, int64_t K, int64_t N,
                                int group, uint8_t* q_out, uint16_t* scales_out,
                                uint8_t* zeros_out, int32_t* bad_zeros, void* stream) {
  using namespace fmoe::repack;
  if (format != FMOE_INT4_AWQ && format != FMOE_INT4_GPTQ_V1 && format != FMOE_INT4_GPTQ_V2)
    return fmoe_host::fail(FMOE_ERR_INVALID, "repack_int4: unknown format %d", format);
  if (!qweight || !qzeros || !scales || !q_out || !scales_out || !zeros_out)
    return fmoe_host::fail(FMOE_ERR_INVALID, "repack_int4: null pointer");
  if (E < 1 || K < 1 || N < 1 || group < 8)
    return fmoe_host::fail(FMOE_ERR_INVALID, "repack_int4: bad sizes E=%lld K=%lld N=%lld group=%d",
                           static_cast<long long>(E), static_cast<long long>(K),
                           static_cast<long long>(N), group);
  if (N % 8 || K % 8 || group % 8 || K % group)
    return fmoe_host::fail(FMOE_ERR_INVALID,
                           "repack_int4: need N %% 8 == 0, K %% group == 0 and group %% 8 == 0 "
                           "(K=%lld N=%lld group=%d)",
                           static_cast<long long>(K), static_cast<long long>(N), group);
  if (E > 65535 || (N + kTile - 1) / kTile > 0x7fffffff || (K + kTile - 1) / kTile > 65535)
    return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "repack_int4: tensor too large for one launch");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned gx = static_cast<unsigned>((N + kTile - 1) / kTile);
  if (format == FMOE_INT4_AWQ) {
    constexpr int TK = kAwqTK, TN = kAwqTN;
    const dim3 g(static_cast<unsigned>((N + TN - 1) / TN), static_cast<unsigned>((K + TK - 1) / TK),
                 static_cast<unsigned>(E));
    awq_weight_kernel<TK, TN><<<g, kThreads, 0, s>>>(qweight, K, N, q_out);
  } else {
    const int64_t K8 = K / 8;
    const dim3 g(gx, static_cast<unsigned>((K8 + kTile - 1) / kTile), static_cast<unsigned>(E));
    gptq_weight_kernel<<<g, kThreads, 0, s>>>(reinterpret_cast<const uint32_t*>(qweight), K8, N,
                                              reinterpret_cast<uint32_t*>(q_out));
  }
  int st = fmoe_host::check_launch("repack_int4 weights");
  if (st != FMOE_OK) return st;
  const int64_t pairs = E * (K / group) * (N / 2);
  const int64_t blocks = (pairs + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "repack_int4: too many groups");
  zeros_scales_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(
      format, reinterpret_cast<const uint32_t*>(qzeros), scales, pairs, N, zeros_out, scales_out,
      bad_zeros);
  return fmoe_host::check_launch("repack_int4 zeros");
}

extern "C" int fmoe_tile_int4(const uint8_t* q, int64_t E, int64_t R, int64_t K, uint8_t* out,
                              void* stream) {
  using namespace fmoe::repack;
  if (!q || !out) return fmoe_host::fail(FMOE_ERR_INVALID, "tile_int4: null pointer");
  if (E < 1 || R < 16 || K < 128 || R % 16 || K % 128)
    return fmoe_host::fail(FMOE_ERR_INVALID,
                           "tile_int4: need E >= 1, R %% 16 == 0 and K %% 128 == 0 (E=%lld R=%lld K=%lld)",
                           static_cast<long long>(E), static_cast<long long>(R), static_cast<long long>(K));
  const int64_t bytes = E * R * (K / 2);
  const uint8_t* qe = q + bytes;
  const uint8_t* oe = out + bytes;
  if (q < oe && out < qe) return fmoe_host::fail(FMOE_ERR_INVALID, "tile_int4: q and out overlap");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out)) % 16)
    return fmoe_host::fail(FMOE_ERR_INVALID, "tile_int4: q and out must be 16-byte aligned");
  const int64_t chunks = bytes / 16;
  const int64_t blocks = (chunks + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "tile_int4: tensor too large");
  tile_int4_kernel<<<static_cast<unsigned>(blocks), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const fmoe::i32x4_t*>(q), chunks, K, reinterpret_cast<fmoe::i32x4_t*>(out));
  return fmoe_host::check_launch("tile_int4");
}

namespace fmoe {
// Device-side helper of the fused large-batch path: 4-bit weights of type
// wtype ([E][R][K] logical) -> bf16 [E][R][K] in out.
int dequant_4bit(int wtype, const void* q, const void* scale, const void* zeros, int64_t E,
                 int64_t R, int64_t K, uint16_t* out, hipStream_t s) {
  using namespace fmoe::repack;
  const bool mx = wtype == FMOE_W_MXFP4 || wtype == FMOE_W_MXFP4_TILED;
  const int tiled = wtype == FMOE_W_INT4_TILED || wtype == FMOE_W_MXFP4_TILED;
  if (!q || !scale || (!mx && !zeros) || !out) return fmoe_host::fail(FMOE_ERR_INVALID, "dequant: null pointer");
  if (R % 16 || K % 128) return fmoe_host::fail(FMOE_ERR_INVALID, "dequant: R %% 16 / K %% 128");
  const int64_t units = E * R * (K / 8);
  const int64_t blocks = (units + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "dequant: tensor too large");
  if (mx)
    dequant_4bit_kernel<true><<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(
        static_cast<const uint8_t*>(q), tiled, scale, nullptr, units, R, K, out);
  else
    dequant_4bit_kernel<false><<<static_cast<unsigned>(blocks), kThreads, 0, s>>>(
        static_cast<const uint8_t*>(q), tiled, scale, static_cast<const uint8_t*>(zeros), units, R, K, out);
  return fmoe_host::check_launch("dequant_4bit");
}
}  // namespace fmoe
