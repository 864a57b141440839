// Router kernels: logits -> (topk_weights, topk_ids).
//
// One wavefront per token; the E scores of a token are spread over the 64
// lanes (up to 16 per lane, E <= 1024) and every selection step is a
// wave-level arg-max over (score, expert) with the lower expert id winning a
// tie.  Selection runs on the logits themselves (softmax and sigmoid are
// monotonic), so the chosen ids do not depend on exp() rounding.
#include "common.hpp"

namespace fmoe {

struct ArgMax {
  float v;
  int i;
};

__device__ __forceinline__ ArgMax wave_argmax(ArgMax a) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float v = __shfl_xor(a.v, o, kWave);
    int i = __shfl_xor(a.i, o, kWave);
    if (v > a.v || (v == a.v && i < a.i)) {
      a.v = v;
      a.i = i;
    }
  }
  return a;
}

// Best (value, index) among this lane's entries; index = lane + 64 * slot.
template <int PL>
__device__ __forceinline__ ArgMax lane_best(const float (&v)[PL], int lane) {
  ArgMax b{-INFINITY, 0x7fffffff};
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    int e = lane + kWave * i;
    if (v[i] > b.v) {  // ascending e within a lane: strict > keeps the lowest id
      b.v = v[i];
      b.i = e;
    }
  }
  return b;
}

template <int PL>
__device__ __forceinline__ void knock_out(float (&v)[PL], int lane, int e) {
#pragma unroll
  for (int i = 0; i < PL; ++i)
    if (lane + kWave * i == e) v[i] = -INFINITY;
}

template <int PL>
__device__ __forceinline__ float pick(const float (&v)[PL], int lane, int e) {
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < PL; ++i)
    if (lane + kWave * i == e) r = v[i];
  return __shfl(r, e % kWave, kWave);
}

// tests/test_fused_moe.py:24-27: softmax over E, top-k, renormalise.
template <int PL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const float* __restrict__ logits,
                                                           int64_t M, int E, int k, int renorm,
                                                           float* __restrict__ w_out,
                                                           int32_t* __restrict__ id_out) {
  const int lane = threadIdx.x % kWave;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (t >= M) return;
  const float* row = logits + t * E;
  float x[PL], p[PL];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    int e = lane + kWave * i;
    x[i] = e < E ? row[e] : -INFINITY;
    mx = fmaxf(mx, x[i]);
  }
  mx = wave_max(mx);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    int e = lane + kWave * i;
    p[i] = e < E ? expf(x[i] - mx) : 0.f;
    s += p[i];
  }
  s = wave_sum(s);
#pragma unroll
  for (int i = 0; i < PL; ++i) p[i] = p[i] / s;

  float myw = 0.f;
  int myid = 0;
  float wsum = 0.f;
  for (int j = 0; j < k; ++j) {
    ArgMax b = wave_argmax(lane_best<PL>(x, lane));
    float pj = pick<PL>(p, lane, b.i);
    wsum += pj;
    if (lane == j) {
      myw = pj;
      myid = b.i;
    }
    knock_out<PL>(x, lane, b.i);
  }
  if (lane < k) {
    w_out[t * k + lane] = renorm ? myw / wsum : myw;
    id_out[t * k + lane] = myid;
  }
}

// DeepSeek-V3 grouped top-k (SGLang biased_grouped_topk semantics).
template <int PL>
__global__ __launch_bounds__(256) void grouped_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int64_t M, int E, int k,
    int n_group, int topk_group, int scoring, int renorm, float* __restrict__ w_out,
    int32_t* __restrict__ id_out) {
  __shared__ float sel_lds[4][1024];
  const int lane = threadIdx.x % kWave;
  const int wid = threadIdx.x / kWave;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + wid;
  // Waves past the last token still run (clamped to token 0) so that every
  // wave reaches the barrier below; they store nothing.
  const bool live = t < M;
  const float* row = logits + (live ? t : 0) * E;
  float sc[PL], sel[PL];
  if (scoring == 0) {
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      int e = lane + kWave * i;
      sc[i] = e < E ? 1.0f / (1.0f + expf(-row[e])) : 0.f;
    }
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      int e = lane + kWave * i;
      sc[i] = e < E ? row[e] : -INFINITY;
      mx = fmaxf(mx, sc[i]);
    }
    mx = wave_max(mx);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      int e = lane + kWave * i;
      sc[i] = e < E ? expf(sc[i] - mx) : 0.f;
      s += sc[i];
    }
    s = wave_sum(s);
#pragma unroll
    for (int i = 0; i < PL; ++i) sc[i] = sc[i] / s;
  }
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    int e = lane + kWave * i;
    sel[i] = e < E ? sc[i] + (bias ? bias[e] : 0.f) : -INFINITY;
    if (e < E) sel_lds[wid][e] = sel[i];
  }
  __syncthreads();
  // group score: sum of the two best biased scores of the group
  const int gsz = E / n_group;
  float gs = -INFINITY;
  if (lane < n_group) {
    float b0 = -INFINITY, b1 = -INFINITY;
    for (int j = 0; j < gsz; ++j) {
      float v = sel_lds[wid][lane * gsz + j];
      if (v > b0) {
        b1 = b0;
        b0 = v;
      } else if (v > b1) {
        b1 = v;
      }
    }
    gs = b0 + b1;
  }
  // keep the topk_group best groups
  uint64_t keep = 0;
  for (int j = 0; j < topk_group; ++j) {
    ArgMax a = wave_argmax(ArgMax{gs, lane});
    keep |= 1ull << a.i;
    if (lane == a.i) gs = -INFINITY;
  }
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    int e = lane + kWave * i;
    if (e < E && !((keep >> (e / gsz)) & 1ull)) sel[i] = -INFINITY;
  }
  float myw = 0.f, wsum = 0.f;
  int myid = 0;
  for (int j = 0; j < k; ++j) {
    ArgMax b = wave_argmax(lane_best<PL>(sel, lane));
    float wj = pick<PL>(sc, lane, b.i);
    wsum += wj;
    if (lane == j) {
      myw = wj;
      myid = b.i;
    }
    knock_out<PL>(sel, lane, b.i);
  }
  if (live && lane < k) {
    w_out[t * k + lane] = renorm ? myw / wsum : myw;
    id_out[t * k + lane] = myid;
  }
}

}  // namespace fmoe

using namespace fmoe;
using fmoe_host::check_launch;
using fmoe_host::fail;

namespace {
int per_lane(int E) {
  int pl = (E + kWave - 1) / kWave;
  if (pl <= 1) return 1;
  if (pl <= 2) return 2;
  if (pl <= 4) return 4;
  if (pl <= 8) return 8;
  return 16;
}
}  // namespace

extern "C" int fmoe_topk_softmax(const float* logits, int64_t M, int E, int k, int renormalize,
                                 float* topk_weights, int32_t* topk_ids, void* stream) {
  if (M < 0 || E < 1 || E > 1024 || k < 1 || k > 32 || k > E)
    return fail(FMOE_ERR_INVALID, "topk_softmax: need 1 <= k <= min(E, 32), E <= 1024 (E=%d k=%d)", E, k);
  if (M == 0) return FMOE_OK;
  if (!logits || !topk_weights || !topk_ids) return fail(FMOE_ERR_INVALID, "topk_softmax: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>((M + 3) / 4)), block(256);
  switch (per_lane(E)) {
#define L(PL) \
  case PL: topk_softmax_kernel<PL><<<grid, block, 0, s>>>(logits, M, E, k, renormalize, topk_weights, topk_ids); break;
    L(1) L(2) L(4) L(8) L(16)
#undef L
  }
  return check_launch("topk_softmax");
}

extern "C" int fmoe_grouped_topk(const float* logits, const float* bias, int64_t M, int E, int k,
                                 int n_group, int topk_group, int scoring, int renormalize,
                                 float* topk_weights, int32_t* topk_ids, void* stream) {
  if (M < 0 || E < 1 || E > 1024 || k < 1 || k > 32 || n_group < 1 || n_group > 64 ||
      E % n_group != 0 || E / n_group < 2 || topk_group < 1 || topk_group > n_group ||
      k > topk_group * (E / n_group) || (scoring != 0 && scoring != 1))
    return fail(FMOE_ERR_INVALID,
                "grouped_topk: bad shape (E=%d k=%d n_group=%d topk_group=%d scoring=%d)", E, k,
                n_group, topk_group, scoring);
  if (M == 0) return FMOE_OK;
  if (!logits || !topk_weights || !topk_ids) return fail(FMOE_ERR_INVALID, "grouped_topk: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>((M + 3) / 4)), block(256);
  switch (per_lane(E)) {
#define L(PL)                                                                                   \
  case PL:                                                                                      \
    grouped_topk_kernel<PL><<<grid, block, 0, s>>>(logits, bias, M, E, k, n_group, topk_group, \
                                                   scoring, renormalize, topk_weights, topk_ids); \
    break;
    L(1) L(2) L(4) L(8) L(16)
#undef L
  }
  return check_launch("grouped_topk");
}
