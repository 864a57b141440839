// Bandwidth-bound helpers of the fused path:
//   * dynamic per-token-group fp8 (e4m3fn) quantization of bf16 rows;
//   * the deterministic top-k combine (moe_sum).
#include "common.hpp"

namespace fmoe {

// One thread = 8 consecutive bf16 (one 16-byte load); `group / 8` threads
// cooperate on a group and reduce its amax with xor-shuffles.
template <int GROUP>
__global__ __launch_bounds__(256) void quant_fp8_group_kernel(const uint16_t* __restrict__ x,
                                                              int64_t n_vec, int64_t K,
                                                              uint8_t* __restrict__ q,
                                                              float* __restrict__ scale) {
  constexpr int TPG = GROUP / 8;  // threads per group
  const int64_t v = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool live = v < n_vec;
  const int64_t vv = live ? v : 0;
  i32x4_t raw = *reinterpret_cast<const i32x4_t*>(x + vv * 8);
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w = static_cast<uint32_t>(raw[i]);
    f[2 * i] = __uint_as_float(w << 16);
    f[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
#pragma unroll
  for (int o = TPG / 2; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, kWave));
  const float s = fmaxf(amax, kFp8Eps) / kFp8Max;
  const float inv = 1.0f / s;
  const uint32_t lo = pack_e4m3x4(fp8_qdiv(f[0], s, inv), fp8_qdiv(f[1], s, inv),
                                  fp8_qdiv(f[2], s, inv), fp8_qdiv(f[3], s, inv));
  const uint32_t hi = pack_e4m3x4(fp8_qdiv(f[4], s, inv), fp8_qdiv(f[5], s, inv),
                                  fp8_qdiv(f[6], s, inv), fp8_qdiv(f[7], s, inv));
  if (!live) return;
  *reinterpret_cast<uint2*>(q + vv * 8) = make_uint2(lo, hi);
  if ((threadIdx.x % TPG) == 0) {
    const int64_t row = (vv * 8) / K, col = (vv * 8) % K;
    scale[row * (K / GROUP) + col / GROUP] = s;
  }
}

// out[t, c] = bf16(scale * sum_j sum_p y[p][gate_indx[t*k+j], c]): the
// token's k slots in ascending j, each slot's split planes in ascending p,
// one running fp32 sum per column in exactly that order (deterministic).
// One thread = 4 columns (16-byte loads).  The (j, p) terms are taken BATCH
// at a time: first every term's slot (the gate_indx loads together), then
// every term's row load -- dropped slots read a row that exists and is not
// added -- so the loads of a batch are in flight together; then the adds in
// order.  (Large calls; decode-size calls go to moe_sum_planes_kernel.)
constexpr int kSumThreads = 256;

template <typename YT>
__device__ __forceinline__ void load4(const YT* src, float (&v)[4]) {
  if constexpr (sizeof(YT) == 4) {
    const float4 f = *reinterpret_cast<const float4*>(src);
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  } else {  // bf16 rows
    const uint2 w = *reinterpret_cast<const uint2*>(src);
    v[0] = __uint_as_float(w.x << 16);
    v[1] = __uint_as_float(w.x & 0xffff0000u);
    v[2] = __uint_as_float(w.y << 16);
    v[3] = __uint_as_float(w.y & 0xffff0000u);
  }
}

template <typename YT, int BATCH>
__global__ __launch_bounds__(kSumThreads) void moe_sum_kernel(const YT* __restrict__ y, int splits,
                                                              int64_t split_stride,
                                                              const int32_t* __restrict__ gate_indx,
                                                              const int32_t* __restrict__ ids, int n_experts,
                                                              int64_t n_tok, int k, int64_t K, float scale,
                                                              uint16_t* __restrict__ out) {
  const int64_t c = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (c >= K) return;
  const int n_terms = k * splits;
  // tokens t = blockIdx.y, blockIdx.y + gridDim.y, ... (grid y is capped at 65535)
  for (int64_t t = blockIdx.y; t < n_tok; t += gridDim.y) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int b = 0; b < n_terms; b += BATCH) {
      // slot of each term: tiny-batch path (gate_indx null) = flat index t k
      // + j, dropped when its expert id is out of range; else gate_indx (< 0:
      // dropped)
      int row[BATCH];
      bool live[BATCH];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int q = b + u;
        live[u] = false;
        row[u] = static_cast<int>(t * k);
        if (q < n_terms) {
          const int64_t f = t * k + q / splits;
          int sl;
          if (gate_indx) {
            sl = gate_indx[f];
          } else {
            const int id = ids[f];
            sl = id >= 0 && id < n_experts ? static_cast<int>(f) : -1;
          }
          live[u] = sl >= 0;
          if (sl >= 0) row[u] = sl;  // else a row that exists, not added
        }
      }
      float v[BATCH][4];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int q = b + u;  // uniform: terms past the last one issue no load
        if (q < n_terms) load4(y + (q % splits) * split_stride + static_cast<int64_t>(row[u]) * K + c, v[u]);
      }
#pragma unroll
      for (int u = 0; u < BATCH; ++u)
        if (live[u]) {
          acc[0] += v[u][0];
          acc[1] += v[u][1];
          acc[2] += v[u][2];
          acc[3] += v[u][3];
        }
    }
    const uint32_t w0 = f32_to_bf16(acc[0] * scale) | (static_cast<uint32_t>(f32_to_bf16(acc[1] * scale)) << 16);
    const uint32_t w1 = f32_to_bf16(acc[2] * scale) | (static_cast<uint32_t>(f32_to_bf16(acc[3] * scale)) << 16);
    *reinterpret_cast<uint2*>(out + t * K + c) = make_uint2(w0, w1);
  }
}

// Top-k sum of one plane of bf16 rows (prefill GEMM2 without split-K, the
// fused path): one wave per token, lane l owning 8-column chunks l, l + 64,
// ...; for each pair of chunks the rows of up to 8 terms are all requested
// (16-byte loads) before the adds, which run in term order j = 0..k-1 per
// column -- moe_sum_kernel's order, so results are bit-identical.  Slots come
// from gate_indx (< 0: dropped, a valid row is read and not added).  k <= 64.
__global__ __launch_bounds__(256) void moe_sum_rows_bf16_kernel(const uint16_t* __restrict__ y,
                                                                const int32_t* __restrict__ gate_indx,
                                                                int64_t n_tok, int k, int64_t K,
                                                                float scale, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x % kWave;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (t >= n_tok) return;
  const int64_t nchunk = K / 8;
  const int my = lane < k ? gate_indx[t * k + lane] : -1;
  for (int64_t c0 = lane; c0 < nchunk; c0 += 2 * kWave) {
    float acc[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
    const bool c1 = c0 + kWave < nchunk;
    for (int j0 = 0; j0 < k; j0 += 8) {
      i32x4_t v[2][8];
      bool ok[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u;
        const int row = __shfl(my, j < k ? j : 0, kWave);
        ok[u] = j < k && row >= 0;
        const uint16_t* src = y + static_cast<int64_t>(row >= 0 ? row : 0) * K + c0 * 8;
        if (j < k) {
          v[0][u] = *reinterpret_cast<const i32x4_t*>(src);
          if (c1) v[1][u] = *reinterpret_cast<const i32x4_t*>(src + kWave * 8);
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (!ok[u]) continue;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (h == 1 && !c1) continue;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t w = static_cast<uint32_t>(v[h][u][q]);
            acc[h][2 * q] += __uint_as_float(w << 16);
            acc[h][2 * q + 1] += __uint_as_float(w & 0xffff0000u);
          }
        }
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 1 && !c1) continue;
      i32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = static_cast<int>(f32_to_bf16(acc[h][2 * q] * scale) |
                                (static_cast<uint32_t>(f32_to_bf16(acc[h][2 * q + 1] * scale)) << 16));
      *reinterpret_cast<i32x4_t*>(out + t * K + (c0 + h * kWave) * 8) = o;
    }
  }
}

// Small calls (decode) use 64-thread blocks, so their few workgroups spread
// over more CUs (each CU keeps only so many loads in flight); most of them go
// to moe_sum_planes_kernel instead (small_sum).
inline void sum_launch_dims(int64_t K, int64_t M, dim3& g, dim3& b) {
  const int64_t vecs = K / 4;
  const int threads = vecs * M < 64 * 1024 ? 64 : kSumThreads;
  g = dim3(static_cast<unsigned>((vecs + threads - 1) / threads), static_cast<unsigned>(M < 65535 ? M : 65535));
  b = dim3(static_cast<unsigned>(threads));
}

// Top-k combine of small calls (decode) and of the one-launch int4 decode's
// N / 128 planes: the terms of an output element, (slot j, plane p), are
// split over 16 term groups g -- planes p = g, g + 16, ... of every slot when
// there are >= 16 planes, else terms q = j * planes + p = g, g + 16, ... --
// each group summed in ascending q, and the 16 group sums are added in order
// g = 0..15: a fixed order per shape, so every run is bit-identical.  A
// workgroup = one token x 64 columns: thread (g, quad) loads its terms for 4
// columns 8 at a time (all in flight together), the group sums meet in LDS.  Slots:
// gate_indx (< 0: dropped) or, with gate_indx null, flat slots t k + j whose
// expert id is in [0, n_experts).
constexpr int kPlaneGroups = 16;
__global__ __launch_bounds__(256) void moe_sum_planes_kernel(const float* __restrict__ y, int planes,
                                                             int64_t plane_stride,
                                                             const int32_t* __restrict__ gate_indx,
                                                             const int32_t* __restrict__ ids, int n_experts,
                                                             int k, int64_t K, float scale,
                                                             uint16_t* __restrict__ out) {
  __shared__ int rows[32];
  __shared__ float4 part[kPlaneGroups][16];
  const int tid = threadIdx.x, quad = tid & 15, g = tid >> 4;
  const int64_t t = blockIdx.y;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + quad * 4;
  if (tid < k) {
    const int64_t f = t * k + tid;
    int sl;
    if (gate_indx) {
      sl = gate_indx[f];
    } else {
      const int id = ids[f];
      sl = id >= 0 && id < n_experts ? static_cast<int>(f) : -1;
    }
    rows[tid] = sl;
  }
  __syncthreads();
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  auto add = [&](const float4& v) {
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  };
  if (planes >= kPlaneGroups) {
    // many planes (one-launch int4 decode): slot by slot, group g taking
    // planes g, g + 16, ... -- q = j * planes + p order within the group
    const int per = (planes - g + kPlaneGroups - 1) / kPlaneGroups;
    for (int j = 0; j < k; ++j) {
      const int row = rows[j];
      if (row < 0) continue;
      const float* src = y + static_cast<int64_t>(row) * K + c + static_cast<int64_t>(g) * plane_stride;
      for (int i0 = 0; i0 < per; i0 += 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (i0 + u < per)
            v[u] = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(i0 + u) * kPlaneGroups * plane_stride);
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (i0 + u < per) add(v[u]);
      }
    }
  } else {
    // few planes (split-K of the decode GEMM2): the k x planes terms dealt
    // round robin over the 16 groups, 8 loads in flight per thread
    const int n_terms = k * planes;
    int tj = g / planes, tp = g - tj * planes;  // (j, p) of term q, stepped without a division
    for (int q0 = g; q0 < n_terms; q0 += 8 * kPlaneGroups) {
      float4 v[8];
      bool ok[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int q = q0 + u * kPlaneGroups;
        ok[u] = false;
        if (q < n_terms) {
          const int row = rows[tj];
          if (row >= 0) {
            v[u] = *reinterpret_cast<const float4*>(y + static_cast<int64_t>(tp) * plane_stride +
                                                    static_cast<int64_t>(row) * K + c);
            ok[u] = true;
          }
          for (tp += kPlaneGroups; tp >= planes; tp -= planes) ++tj;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (ok[u]) add(v[u]);
    }
  }
  part[g][quad] = acc;
  __syncthreads();
  if (g != 0) return;
  float4 sum = part[0][quad];
  for (int h = 1; h < kPlaneGroups; ++h) {
    const float4 v = part[h][quad];
    sum.x += v.x;
    sum.y += v.y;
    sum.z += v.z;
    sum.w += v.w;
  }
  const uint32_t w0 = f32_to_bf16(sum.x * scale) | (static_cast<uint32_t>(f32_to_bf16(sum.y * scale)) << 16);
  const uint32_t w1 = f32_to_bf16(sum.z * scale) | (static_cast<uint32_t>(f32_to_bf16(sum.w * scale)) << 16);
  *reinterpret_cast<uint2*>(out + t * K + c) = make_uint2(w0, w1);
}

}  // namespace fmoe

using namespace fmoe;
using fmoe_host::check_launch;
using fmoe_host::fail;

extern "C" int fmoe_quant_fp8_group(const void* x, int64_t M, int64_t K, int group, void* q,
                                    float* scale, void* stream) {
  if (M < 0 || K <= 0 || (group != 64 && group != 128) || K % group != 0)
    return fail(FMOE_ERR_INVALID, "quant_fp8_group: need K %% group == 0, group in {64,128} (K=%lld group=%d)",
                static_cast<long long>(K), group);
  if (M == 0) return FMOE_OK;
  if (!x || !q || !scale) return fail(FMOE_ERR_INVALID, "quant_fp8_group: null pointer");
  const int64_t n_vec = M * K / 8;
  dim3 g(static_cast<unsigned>((n_vec + 255) / 256)), b(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (group == 128)
    quant_fp8_group_kernel<128><<<g, b, 0, s>>>(static_cast<const uint16_t*>(x), n_vec, K,
                                                static_cast<uint8_t*>(q), scale);
  else
    quant_fp8_group_kernel<64><<<g, b, 0, s>>>(static_cast<const uint16_t*>(x), n_vec, K,
                                               static_cast<uint8_t*>(q), scale);
  return check_launch("quant_fp8_group");
}

namespace fmoe {
int moe_sum_planes(const float* y, int planes, const int32_t* gate_indx, const int32_t* ids, int E,
                   int64_t M, int k, int64_t K, float scale, void* out, hipStream_t s);
// Small calls (decode: fewer than 64K column quads) take the term-parallel
// kernel: their few tokens leave most CUs idle and the per-thread term loop's
// round trips would set the time (reference sweep M=1: 48 terms per element).
bool small_sum(int64_t K, int64_t M, int k) {
  return K % 64 == 0 && k <= 32 && M <= 65535 && (K / 4) * M < 64 * 1024;
}
}  // namespace fmoe

extern "C" int fmoe_moe_sum(const float* y, int splits, const int32_t* gate_indx, int64_t M, int k,
                            int64_t K, float scale, void* out, void* stream) {
  if (M < 0 || k < 1 || K <= 0 || K % 4 != 0 || splits < 1)
    return fail(FMOE_ERR_INVALID, "moe_sum: need K %% 4 == 0, k >= 1, splits >= 1");
  if (M == 0) return FMOE_OK;
  if (!y || !gate_indx || !out) return fail(FMOE_ERR_INVALID, "moe_sum: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (small_sum(K, M, k)) return moe_sum_planes(y, splits, gate_indx, nullptr, 0, M, k, K, scale, out, s);
  dim3 g, b;
  sum_launch_dims(K, M, g, b);
  moe_sum_kernel<float, 8><<<g, b, 0, s>>>(y, splits, M * k * K, gate_indx, nullptr, 0, M, k, K, scale,
                                           static_cast<uint16_t*>(out));
  return check_launch("moe_sum");
}

namespace fmoe {
// moe_sum of the tiny-batch decode path: y rows are flat slots (t * k + j).
int moe_sum_flat(const float* y, int splits, const int32_t* ids, int E, int64_t M, int k, int64_t K,
                 float scale, void* out, hipStream_t s) {
  if (small_sum(K, M, k)) return moe_sum_planes(y, splits, nullptr, ids, E, M, k, K, scale, out, s);
  dim3 g, b;
  sum_launch_dims(K, M, g, b);
  moe_sum_kernel<float, 8><<<g, b, 0, s>>>(y, splits, M * k * K, nullptr, ids, E, M, k, K, scale,
                                           static_cast<uint16_t*>(out));
  return check_launch("moe_sum");
}
// moe_sum over one plane of bf16 y rows (prefill GEMM2 without split-K).
int moe_sum_bf16(const uint16_t* y, const int32_t* gate_indx, int64_t M, int k, int64_t K,
                 float scale, void* out, hipStream_t s) {
  if (k <= kWave && K % 8 == 0) {
    const dim3 g(static_cast<unsigned>((M + 3) / 4)), b(256);
    moe_sum_rows_bf16_kernel<<<g, b, 0, s>>>(y, gate_indx, M, k, K, scale, static_cast<uint16_t*>(out));
    return check_launch("moe_sum_rows");
  }
  dim3 g, b;
  sum_launch_dims(K, M, g, b);
  moe_sum_kernel<__bf16, 8><<<g, b, 0, s>>>(reinterpret_cast<const __bf16*>(y), 1, M * k * K, gate_indx,
                                         nullptr, 0, M, k, K, scale, static_cast<uint16_t*>(out));
  return check_launch("moe_sum");
}
// moe_sum_planes_kernel over `planes` split planes (gate_indx, or flat slots
// checked against the expert ids when gate_indx is null).
int moe_sum_planes(const float* y, int planes, const int32_t* gate_indx, const int32_t* ids, int E,
                   int64_t M, int k, int64_t K, float scale, void* out, hipStream_t s) {
  if (k > 32 || K % 64 != 0 || M > 65535)
    return fmoe_host::fail(FMOE_ERR_UNSUPPORTED, "moe_sum_planes: k <= 32, K %% 64 == 0, M <= 65535");
  const dim3 g(static_cast<unsigned>(K / 64), static_cast<unsigned>(M)), b(256);
  moe_sum_planes_kernel<<<g, b, 0, s>>>(y, planes, M * k * K, gate_indx, ids, E, k, K, scale,
                                        static_cast<uint16_t*>(out));
  return check_launch("moe_sum_planes");
}
}  // namespace fmoe
