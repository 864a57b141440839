// moe_align: top-k routing -> expert-sorted slot order, ExptData tile map and
// SGLang's padded sorted_token_ids, bit-exact and deterministic.
//
// Replaces _standard_topk_to_triton_kernels (ops/fused_moe.py:103-130) and
// the compute_expt_data_torch call at :124.  Three phases over chunks of 256
// tokens (k*256 slots):
//   rows    per token: order its k ids ascending (rank by counting, ties by
//           column), write expt_indx / expt_scal, count the chunk's per-expert
//           histogram in LDS;
//   scan    per expert, exclusive prefix over chunks, then the exclusive
//           scan over experts (token_offs_raw), the padded tile offsets
//           (token_offs_pad) and the tile map -- recomputed by every scatter
//           workgroup from the chunk histograms (integer sums, so all agree);
//   scatter per chunk, in slot order: a slot's rank among equal experts is
//           found with wave ballots (no atomics decide a position), so each
//           expert's slots keep ascending flat order — the stable argsort of
//           :118 — and every run writes identical bits.
// Two launches (rows, scan + scatter); for one chunk (M <= 256) the three
// phases run in a single workgroup launch.
#include "common.hpp"

namespace fmoe {

constexpr int kAlignThreads = 256;
constexpr int kMaxExperts = 1024;

struct AlignParams {
  const int32_t* ids;
  const float* w;
  int64_t M;
  int k;
  int E;
  int bm;
  int64_t max_tiles;
  int64_t sorted_cap;  // length of sorted_token_ids
  int n_chunks;
  int32_t* chunk_hist;  // [n_chunks, E]
  int32_t* chunk_base;  // [n_chunks, E]
  int32_t* sort_col;    // [M*k] original column of each row-sorted entry
  fmoe_align_out o;
  const int32_t* emap;  // optional expert map: global id -> local id or -1
  int n_global;
};

// Expert id of flat slot f (global -> local through the expert map, if any;
// ids outside the map, or mapped to -1, are dropped like out-of-range ids).
__device__ __forceinline__ int load_id(const AlignParams& p, int64_t f) {
  int v = p.ids[f];
  if (p.emap) v = (v >= 0 && v < p.n_global) ? p.emap[v] : -1;
  return v;
}

// A chunk holds at most 256 tokens x 32 slots.
constexpr int kChunkSlots = kAlignThreads * 32;

// Workgroup barrier that orders LDS only.  Around it the chunked phases store
// to global addresses that no other thread of the launch reads, so those
// stores need not drain at every barrier (__syncthreads waits for them).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Copy n consecutive 4-byte values src[0..n) into LDS dst[0..n) (coalesced,
// 8 loads per thread in flight).  load(i) returns the value of slot i.
template <typename T, typename Load>
__device__ __forceinline__ void stage_chunk(T* dst, int n, Load load) {
  const int tid = threadIdx.x;
  for (int i0 = 0; i0 < n; i0 += 8 * kAlignThreads) {
    T v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * kAlignThreads + tid;
      v[u] = i < n ? load(i) : T(0);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * kAlignThreads + tid;
      if (i < n) dst[i] = v[u];
    }
  }
}

// Number of slots in chunk c (256 tokens, the last one partial).
__device__ __forceinline__ int chunk_slots(const AlignParams& p, int c) {
  const int64_t f0 = static_cast<int64_t>(c) * kAlignThreads * p.k;
  const int64_t left = p.M * p.k - f0;
  return static_cast<int>(left < kAlignThreads * p.k ? left : kAlignThreads * p.k);
}

// ---- phase 1: per-token sort + chunk histogram.  The chunk's ids and
// weights are staged in LDS first, so each token's k x k rank comparisons
// read LDS instead of issuing one dependent global load each.
__device__ void phase_rows(const AlignParams& p, int c, int* h, int* s_id, float* s_w) {
  const int tid = threadIdx.x;
  for (int e = tid; e < p.E; e += kAlignThreads) h[e] = 0;
  const int64_t f0 = static_cast<int64_t>(c) * kAlignThreads * p.k;
  const int n = chunk_slots(p, c);
  stage_chunk(s_id, n, [&](int i) { return load_id(p, f0 + i); });
  stage_chunk(s_w, n, [&](int i) { return p.w[f0 + i]; });
  lds_barrier();
  const int64_t t = static_cast<int64_t>(c) * kAlignThreads + tid;
  if (t < p.M) {
    const int* row = s_id + tid * p.k;
    const float* wr = s_w + tid * p.k;
    for (int j = 0; j < p.k; ++j) {
      const int idj = row[j];
      int rank = 0;
      for (int i = 0; i < p.k; ++i) {
        const int idi = row[i];
        rank += (idi < idj) || (idi == idj && i < j);
      }
      const int64_t f = t * p.k + rank;
      p.o.expt_indx[f] = idj;
      p.o.expt_scal[f] = wr[j];
      p.sort_col[f] = j;
      if (idj >= 0 && idj < p.E) atomicAdd(&h[idj], 1);
    }
  }
  lds_barrier();
  for (int e = tid; e < p.E; e += kAlignThreads) p.chunk_hist[static_cast<int64_t>(c) * p.E + e] = h[e];
}

// Exclusive scan of one value per thread over the 256-thread block.
__device__ int block_exclusive_scan(int v, int* lds_tmp, int* total) {
  const int lane = threadIdx.x % kWave, wid = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == kWave - 1) lds_tmp[wid] = x;
  lds_barrier();
  int wbase = 0, tot = 0;
  for (int i = 0; i < kAlignThreads / kWave; ++i) {
    int s = lds_tmp[i];
    if (i < wid) wbase += s;
    tot += s;
  }
  lds_barrier();
  *total = tot;
  return wbase + x - v;
}

// Tile map (ExptData.block_pid_map) and SGLang expert_ids from the padded
// tile offsets in LDS: tile tt belongs to the last expert whose offset <= tt.
// Entries tt = first, first + stride, ... are written by this workgroup.
__device__ void write_tile_map(const AlignParams& p, const int* offs_pad_lds, int ttot,
                               int64_t first = -1, int64_t stride = kAlignThreads) {
  const int64_t nblk_cap = p.o.expert_ids ? p.sorted_cap / p.bm + 1 : 0;
  const int64_t lim = p.max_tiles > nblk_cap ? p.max_tiles : nblk_cap;
  for (int64_t tt = first < 0 ? threadIdx.x : first; tt < lim; tt += stride) {
    int val = -1, ex = -1;
    if (tt < ttot) {
      int lo = 0, hi = p.E;  // offs_pad_lds[lo] <= tt < offs_pad_lds[hi]
      while (hi - lo > 1) {
        int mid = (lo + hi) >> 1;
        if (offs_pad_lds[mid] <= tt) lo = mid; else hi = mid;
      }
      ex = lo;
      val = (static_cast<int>(tt - offs_pad_lds[lo]) << 16) | lo;
    }
    if (tt < p.max_tiles) p.o.tile_map[tt] = val;
    if (tt < nblk_cap) p.o.expert_ids[tt] = ex;
  }
}

// ---- phase 2: prefix over chunks and experts, ExptData, SGLang block ids.
// hist_in != nullptr: histogram given directly (fmoe_expt_data); no chunks.
__device__ void phase_scan(const AlignParams& p, const int32_t* hist_in, int* offs_pad_lds,
                           int* tmp) {
  const int tid = threadIdx.x;
  constexpr int PER = kMaxExperts / kAlignThreads;  // experts per thread
  int hv[PER], tv[PER];
  int hsum = 0, tsum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) hv[i] = 0;
  if (hist_in) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid * PER + i;
      if (e < p.E) hv[i] = hist_in[e];
    }
  } else {
    // per expert, exclusive prefix over the chunks: the loads of kBatch
    // chunks x PER experts are issued together (the chunk_base stores
    // cannot alias them), instead of one dependent round trip per chunk
    constexpr int kBatch = 8;
    const int32_t* __restrict__ ch = p.chunk_hist;
    int32_t* __restrict__ cb = p.chunk_base;
    for (int c0 = 0; c0 < p.n_chunks; c0 += kBatch) {
      int v[kBatch][PER];
#pragma unroll
      for (int b = 0; b < kBatch; ++b)
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int e = tid * PER + i;
          v[b][i] = (c0 + b < p.n_chunks && e < p.E) ? ch[static_cast<int64_t>(c0 + b) * p.E + e] : 0;
        }
#pragma unroll
      for (int b = 0; b < kBatch; ++b)
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int e = tid * PER + i;
          if (c0 + b < p.n_chunks && e < p.E) cb[static_cast<int64_t>(c0 + b) * p.E + e] = hv[i];
          hv[i] += v[b][i];
        }
    }
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    tv[i] = (hv[i] + p.bm - 1) / p.bm;
    hsum += hv[i];
    tsum += tv[i];
  }
  int htot, ttot;
  int hbase = block_exclusive_scan(hsum, tmp, &htot);
  int tbase = block_exclusive_scan(tsum, tmp, &ttot);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    int e = tid * PER + i;
    if (e < p.E) {
      if (p.o.hist) p.o.hist[e] = hv[i];
      p.o.offs_raw[e] = hbase;
      p.o.offs_pad[e] = tbase;
      offs_pad_lds[e] = tbase;
    }
    hbase += hv[i];
    tbase += tv[i];
  }
  if (tid == 0) {
    p.o.offs_raw[p.E] = htot;
    p.o.offs_pad[p.E] = ttot;
    offs_pad_lds[p.E] = ttot;
    p.o.n_tiles[0] = ttot;
    if (p.o.num_tokens_post_padded) p.o.num_tokens_post_padded[0] = ttot * p.bm;
  }
  __syncthreads();
  write_tile_map(p, offs_pad_lds, ttot);
}

// ---- phase 2b (chunked path, inside the scatter launch): every scatter
// workgroup recomputes the scan from the chunk histograms (C x E integers,
// read in batches), so no separate one-workgroup scan launch sits between
// rows and scatter.  Integer sums: every workgroup gets the same offsets,
// identical to phase_scan's.  Workgroup c keeps in LDS, per expert, its
// chunk's first slot position (base) and the padded-order shift (padshift);
// workgroup 0 writes ExptData / histogram outputs, and all workgroups share
// the tile map.
__device__ void phase_scan_local(const AlignParams& p, int c, int* base, int* padshift,
                                 int* offs_pad_lds, int* tmp) {
  const int tid = threadIdx.x;
  constexpr int PER = kMaxExperts / kAlignThreads;
  int hv[PER], bv[PER], tv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) hv[i] = bv[i] = 0;
  constexpr int kBatch = 8;
  const int32_t* __restrict__ ch = p.chunk_hist;
  for (int c0 = 0; c0 < p.n_chunks; c0 += kBatch) {
    int v[kBatch][PER];
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int e = tid * PER + i;
        v[b][i] = (c0 + b < p.n_chunks && e < p.E) ? ch[static_cast<int64_t>(c0 + b) * p.E + e] : 0;
      }
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        if (c0 + b == c) bv[i] = hv[i];
        hv[i] += v[b][i];
      }
  }
  int hsum = 0, tsum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    tv[i] = (hv[i] + p.bm - 1) / p.bm;
    hsum += hv[i];
    tsum += tv[i];
  }
  int htot, ttot;
  int hbase = block_exclusive_scan(hsum, tmp, &htot);
  int tbase = block_exclusive_scan(tsum, tmp, &ttot);
  const bool lead = c == 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = tid * PER + i;
    if (e < p.E) {
      if (lead) {
        if (p.o.hist) p.o.hist[e] = hv[i];
        p.o.offs_raw[e] = hbase;
        p.o.offs_pad[e] = tbase;
      }
      offs_pad_lds[e] = tbase;
      base[e] = hbase + bv[i];
      padshift[e] = tbase * p.bm - hbase;
    }
    hbase += hv[i];
    tbase += tv[i];
  }
  if (tid == 0) {
    offs_pad_lds[p.E] = ttot;
    if (lead) {
      p.o.offs_raw[p.E] = htot;
      p.o.offs_pad[p.E] = ttot;
      p.o.n_tiles[0] = ttot;
      if (p.o.num_tokens_post_padded) p.o.num_tokens_post_padded[0] = ttot * p.bm;
    }
  }
  lds_barrier();
  write_tile_map(p, offs_pad_lds, ttot, static_cast<int64_t>(c) * kAlignThreads + tid,
                 static_cast<int64_t>(p.n_chunks) * kAlignThreads);
}

// base / padshift of chunk c from the scan outputs in global memory (one
// workgroup that ran phase_scan itself).
__device__ void scatter_bases_from_global(const AlignParams& p, int c, int* base, int* padshift) {
  for (int e = threadIdx.x; e < p.E; e += kAlignThreads) {
    const int ob = p.o.offs_raw[e];
    base[e] = ob + p.chunk_base[static_cast<int64_t>(c) * p.E + e];
    padshift[e] = p.o.offs_pad[e] * p.bm - ob;
  }
}

// ---- phase 3: stable scatter of one chunk (base / padshift already in LDS).
// The chunk's row-sorted ids, weights and source columns are staged in LDS
// first (all loads in flight), so the k ballot rounds touch no global loads.
__device__ void phase_scatter(const AlignParams& p, int c, int* run, int (*wcnt)[kMaxExperts],
                              const int* base, const int* padshift, int* s_e, float* s_scal,
                              int* s_col) {
  const int tid = threadIdx.x, lane = tid % kWave, wid = tid / kWave;
  for (int e = tid; e < p.E; e += kAlignThreads) {
    run[e] = 0;
    for (int w = 0; w < kAlignThreads / kWave; ++w) wcnt[w][e] = 0;
  }
  const int64_t f0 = static_cast<int64_t>(c) * kAlignThreads * p.k;
  const int n = chunk_slots(p, c);
  stage_chunk(s_e, n, [&](int i) { return p.o.expt_indx[f0 + i]; });
  stage_chunk(s_scal, n, [&](int i) { return p.o.expt_scal[f0 + i]; });
  if (p.o.sorted_token_ids) stage_chunk(s_col, n, [&](int i) { return p.sort_col[f0 + i]; });
  lds_barrier();
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int it = 0; it < p.k; ++it) {
    const int i = it * kAlignThreads + tid;
    const int64_t f = f0 + i;
    int e = p.E;  // marker: no expert (past the end, or an out-of-range id)
    if (i < n) {
      int v = s_e[i];
      if (v >= 0 && v < p.E) e = v;
      else p.o.gate_indx[f] = -1;
    }
    // lanes holding the same expert: AND of per-bit ballots (11 bits: E <= 1024)
    uint64_t m = ~0ull;
#pragma unroll
    for (int b = 0; b < 11; ++b) {
      int bit = (e >> b) & 1;
      uint64_t v = __ballot(bit);
      m &= bit ? v : ~v;
    }
    const int r = __popcll(m & lt);
    const int cnt = __popcll(m);
    const bool live = e < p.E;
    const bool leader = live && r == cnt - 1;
    if (leader) wcnt[wid][e] = cnt;
    lds_barrier();
    if (live) {
      int before = run[e];
      for (int w = 0; w < wid; ++w) before += wcnt[w][e];
      const int pos = base[e] + before + r;
      p.o.topk_indx[pos] = static_cast<int32_t>(f);
      p.o.gate_indx[f] = pos;
      p.o.gate_scal[pos] = s_scal[i];
      if (p.o.sorted_token_ids) {
        const int64_t t = f / p.k;
        p.o.sorted_token_ids[pos + padshift[e]] = static_cast<int32_t>(t * p.k + s_col[i]);
      }
    }
    lds_barrier();
    if (leader) {
      atomicAdd(&run[e], cnt);  // integer sum: order-independent
      wcnt[wid][e] = 0;
    }
    lds_barrier();
  }
}

__device__ void fill_sentinel(const AlignParams& p, int64_t start, int64_t stride) {
  if (!p.o.sorted_token_ids) return;
  const int32_t sentinel = static_cast<int32_t>(p.M * p.k);
  for (int64_t i = start; i < p.sorted_cap; i += stride) p.o.sorted_token_ids[i] = sentinel;
}

__global__ __launch_bounds__(kAlignThreads) void align_rows_kernel(AlignParams p) {
  __shared__ int h[kMaxExperts];
  __shared__ int s_id[kChunkSlots];
  __shared__ float s_w[kChunkSlots];
  phase_rows(p, blockIdx.x, h, s_id, s_w);
  fill_sentinel(p, static_cast<int64_t>(blockIdx.x) * kAlignThreads + threadIdx.x,
                static_cast<int64_t>(gridDim.x) * kAlignThreads);
}

__global__ __launch_bounds__(kAlignThreads) void align_scan_kernel(AlignParams p, const int32_t* hist_in) {
  __shared__ int offs_pad_lds[kMaxExperts + 1];
  __shared__ int tmp[kAlignThreads / kWave];
  phase_scan(p, hist_in, offs_pad_lds, tmp);
}

// Scan (recomputed per workgroup) + stable scatter of chunk blockIdx.x.
__global__ __launch_bounds__(kAlignThreads) void align_scatter_kernel(AlignParams p) {
  __shared__ int run[kMaxExperts];
  __shared__ int wcnt[kAlignThreads / kWave][kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int padshift[kMaxExperts];
  __shared__ int offs_pad_lds[kMaxExperts + 1];
  __shared__ int tmp[kAlignThreads / kWave];
  __shared__ int s_e[kChunkSlots];
  __shared__ float s_scal[kChunkSlots];
  __shared__ int s_col[kChunkSlots];
  phase_scan_local(p, blockIdx.x, base, padshift, offs_pad_lds, tmp);
  phase_scatter(p, blockIdx.x, run, wcnt, base, padshift, s_e, s_scal, s_col);
}

// All three phases in one workgroup (one chunk: M <= 256).
__global__ __launch_bounds__(kAlignThreads) void align_small_kernel(AlignParams p) {
  __shared__ int run[kMaxExperts];
  __shared__ int wcnt[kAlignThreads / kWave][kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int padshift[kMaxExperts + 1];
  __shared__ int tmp[kAlignThreads / kWave];
  __shared__ int s_a[kChunkSlots];
  __shared__ float s_b[kChunkSlots];
  __shared__ int s_c[kChunkSlots];
  fill_sentinel(p, threadIdx.x, kAlignThreads);
  phase_rows(p, 0, run, s_a, s_b);
  __syncthreads();
  phase_scan(p, nullptr, padshift, tmp);
  __syncthreads();
  scatter_bases_from_global(p, 0, base, padshift);
  phase_scatter(p, 0, run, wcnt, base, padshift, s_a, s_b, s_c);
}


// Small batches (M*k <= kTinySlots): the three phases in one workgroup with
// every intermediate in LDS (no global round trips between phases).  Same
// outputs, bit for bit, as the chunked path: ranks by counting within a row,
// stable ballot ranks within an expert.
constexpr int kTinySlots = 1024;

__global__ __launch_bounds__(kAlignThreads) void align_tiny_kernel(AlignParams p) {
  __shared__ int s_e[kTinySlots];
  __shared__ int s_col[kTinySlots];
  __shared__ int s_id[kTinySlots];
  __shared__ float s_w[kTinySlots];
  __shared__ int hist[kMaxExperts];
  __shared__ int offs[kMaxExperts + 1];
  __shared__ int offs_pad[kMaxExperts + 1];
  __shared__ int wcnt[kAlignThreads / kWave][kMaxExperts];
  __shared__ int run[kMaxExperts];
  __shared__ int tmp[kAlignThreads / kWave];
  const int tid = threadIdx.x, lane = tid % kWave, wid = tid / kWave;
  const int n = static_cast<int>(p.M * p.k);
  fill_sentinel(p, tid, kAlignThreads);
  for (int e = tid; e < p.E; e += kAlignThreads) {
    hist[e] = 0;
    run[e] = 0;
    for (int w = 0; w < kAlignThreads / kWave; ++w) wcnt[w][e] = 0;
  }
  for (int f = tid; f < n; f += kAlignThreads) {  // coalesced, independent loads
    s_id[f] = load_id(p, f);
    s_w[f] = p.w[f];
  }
  __syncthreads();
  // rows: per-token counting sort of its k ids
  for (int t = tid; t < p.M; t += kAlignThreads) {
    const int* row = s_id + t * p.k;
    const float* wr = s_w + t * p.k;
    for (int j = 0; j < p.k; ++j) {
      const int idj = row[j];
      int rank = 0;
      for (int i = 0; i < p.k; ++i) {
        const int idi = row[i];
        rank += (idi < idj) || (idi == idj && i < j);
      }
      const int f = t * p.k + rank;
      s_e[f] = idj;
      s_col[f] = j;
      p.o.expt_indx[f] = idj;
      p.o.expt_scal[f] = wr[j];
      if (idj >= 0 && idj < p.E) atomicAdd(&hist[idj], 1);
    }
  }
  __syncthreads();
  // scan over experts (4 per thread, E <= 1024)
  constexpr int PER = kMaxExperts / kAlignThreads;
  int hv[PER], tv[PER], hsum = 0, tsum = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = tid * PER + i;
    hv[i] = e < p.E ? hist[e] : 0;
    tv[i] = (hv[i] + p.bm - 1) / p.bm;
    hsum += hv[i];
    tsum += tv[i];
  }
  int htot, ttot;
  int hb = block_exclusive_scan(hsum, tmp, &htot);
  int tb = block_exclusive_scan(tsum, tmp, &ttot);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = tid * PER + i;
    if (e < p.E) {
      offs[e] = hb;
      offs_pad[e] = tb;
      if (p.o.hist) p.o.hist[e] = hv[i];
      p.o.offs_raw[e] = hb;
      p.o.offs_pad[e] = tb;
    }
    hb += hv[i];
    tb += tv[i];
  }
  if (tid == 0) {
    offs[p.E] = htot;
    offs_pad[p.E] = ttot;
    p.o.offs_raw[p.E] = htot;
    p.o.offs_pad[p.E] = ttot;
    p.o.n_tiles[0] = ttot;
    if (p.o.num_tokens_post_padded) p.o.num_tokens_post_padded[0] = ttot * p.bm;
  }
  __syncthreads();
  write_tile_map(p, offs_pad, ttot);
  // stable scatter (ballot ranks within each wave, wave counts through LDS)
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int f0 = 0; f0 < n; f0 += kAlignThreads) {
    const int f = f0 + tid;
    int e = p.E;
    if (f < n) {
      const int v = s_e[f];
      if (v >= 0 && v < p.E) e = v;
      else p.o.gate_indx[f] = -1;
    }
    uint64_t m = ~0ull;
#pragma unroll
    for (int b = 0; b < 11; ++b) {
      const int bit = (e >> b) & 1;
      const uint64_t v = __ballot(bit);
      m &= bit ? v : ~v;
    }
    const int r = __popcll(m & lt);
    const int cnt = __popcll(m);
    const bool live = e < p.E;
    const bool leader = live && r == cnt - 1;
    if (leader) wcnt[wid][e] = cnt;
    __syncthreads();
    if (live) {
      int before = run[e];
      for (int w = 0; w < wid; ++w) before += wcnt[w][e];
      const int pos = offs[e] + before + r;
      p.o.topk_indx[pos] = f;
      p.o.gate_indx[f] = pos;
      p.o.gate_scal[pos] = p.o.expt_scal[f];
      if (p.o.sorted_token_ids)
        p.o.sorted_token_ids[pos + offs_pad[e] * p.bm - offs[e]] = (f / p.k) * p.k + s_col[f];
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&run[e], cnt);
      wcnt[wid][e] = 0;
    }
    __syncthreads();
  }
}
}  // namespace fmoe

using namespace fmoe;
using fmoe_host::check_launch;
using fmoe_host::fail;

namespace {
int64_t n_chunks_for(int64_t M) { return (M + kAlignThreads - 1) / kAlignThreads; }
size_t align_up(size_t v) { return (v + 255) & ~size_t(255); }
}  // namespace

extern "C" int64_t fmoe_max_tiles(int64_t n_slots, int E) {
  // triton_kernels.routing length (smallest tile height 16): one tile per
  // slot while slots <= E, else every non-empty expert may waste a partial tile.
  if (n_slots <= E) return n_slots > 0 ? n_slots : 1;
  return E - 1 + (n_slots - E + 1 + 15) / 16;
}

extern "C" int64_t fmoe_sorted_ids_len(int64_t n_slots, int E, int block_m) {
  return n_slots + static_cast<int64_t>(E) * (block_m - 1);
}

extern "C" size_t fmoe_align_workspace_bytes(int64_t M, int k, int E) {
  const int64_t C = n_chunks_for(M);
  return 2 * align_up(sizeof(int32_t) * C * E) + align_up(sizeof(int32_t) * M * k);
}

extern "C" int fmoe_align(const int32_t* topk_ids, const float* topk_weights, int64_t M, int k,
                          int E, int block_m, const fmoe_align_out* out, void* workspace,
                          size_t workspace_bytes, void* stream) {
  return fmoe_align_ex(topk_ids, topk_weights, M, k, E, block_m, nullptr, 0, out, workspace,
                       workspace_bytes, stream);
}

extern "C" int fmoe_align_ex(const int32_t* topk_ids, const float* topk_weights, int64_t M, int k,
                             int E, int block_m, const int32_t* expert_map, int n_global,
                             const fmoe_align_out* out, void* workspace, size_t workspace_bytes,
                             void* stream) {
  if (!out) return fail(FMOE_ERR_INVALID, "align: null output struct");
  if (expert_map && n_global < 1)
    return fail(FMOE_ERR_INVALID, "align: expert map needs n_global >= 1 (got %d)", n_global);
  if (M < 0 || k < 1 || k > 32 || E < 1 || E > kMaxExperts)
    return fail(FMOE_ERR_INVALID, "align: need 1 <= k <= 32, 1 <= E <= %d (M=%lld k=%d E=%d)",
                kMaxExperts, static_cast<long long>(M), k, E);
  if (block_m != 16 && block_m != 32 && block_m != 64 && block_m != 128 && block_m != 160 && block_m != 256)
    return fail(FMOE_ERR_UNSUPPORTED, "align: block_m=%d is not supported", block_m);
  if (M * k > (int64_t(1) << 31) - 1 || M * k / block_m + E >= (1 << 15))
    return fail(FMOE_ERR_UNSUPPORTED, "align: %lld slots is not supported", static_cast<long long>(M * k));
  const fmoe_align_out& o = *out;
  // per-slot arrays are empty (and may be null) when M == 0
  if ((M > 0 && (!o.expt_indx || !o.expt_scal || !o.topk_indx || !o.gate_indx || !o.gate_scal)) ||
      !o.offs_raw || !o.offs_pad || !o.tile_map || !o.n_tiles)
    return fail(FMOE_ERR_INVALID, "align: a required output pointer is null");
  if (workspace_bytes < fmoe_align_workspace_bytes(M, k, E))
    return fail(FMOE_ERR_WORKSPACE, "align: workspace %zu < %zu bytes", workspace_bytes,
                fmoe_align_workspace_bytes(M, k, E));
  if (M > 0 && (!topk_ids || !topk_weights)) return fail(FMOE_ERR_INVALID, "align: null input");

  AlignParams p{};
  p.ids = topk_ids;
  p.w = topk_weights;
  p.M = M;
  p.k = k;
  p.E = E;
  p.bm = block_m;
  p.max_tiles = fmoe_max_tiles(M * k, E);
  p.sorted_cap = fmoe_sorted_ids_len(M * k, E, block_m);
  p.n_chunks = static_cast<int>(n_chunks_for(M));
  const int64_t C = p.n_chunks;
  char* ws = static_cast<char*>(workspace);
  p.chunk_hist = reinterpret_cast<int32_t*>(ws);
  p.chunk_base = reinterpret_cast<int32_t*>(ws + align_up(sizeof(int32_t) * C * E));
  p.sort_col = reinterpret_cast<int32_t*>(ws + 2 * align_up(sizeof(int32_t) * C * E));
  p.o = o;
  p.emap = expert_map;
  p.n_global = expert_map ? n_global : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (M * k <= kTinySlots) {
    align_tiny_kernel<<<1, kAlignThreads, 0, s>>>(p);
  } else if (C <= 1) {
    align_small_kernel<<<1, kAlignThreads, 0, s>>>(p);
  } else {
    align_rows_kernel<<<static_cast<unsigned>(C), kAlignThreads, 0, s>>>(p);
    align_scatter_kernel<<<static_cast<unsigned>(C), kAlignThreads, 0, s>>>(p);
  }
  return check_launch("align");
}

extern "C" int fmoe_expt_data(const int32_t* hist, int E, int64_t n_slots, int block_m,
                              int32_t* offs_raw, int32_t* offs_pad, int32_t* tile_map,
                              int32_t* n_tiles, void* stream) {
  if (E < 1 || E > kMaxExperts || n_slots < 0)
    return fail(FMOE_ERR_INVALID, "expt_data: need 1 <= E <= %d", kMaxExperts);
  if (block_m != 16 && block_m != 32 && block_m != 64 && block_m != 128 && block_m != 160 && block_m != 256)
    return fail(FMOE_ERR_UNSUPPORTED, "expt_data: block_m=%d is not supported", block_m);
  if (!hist || !offs_raw || !offs_pad || !tile_map || !n_tiles)
    return fail(FMOE_ERR_INVALID, "expt_data: null pointer");
  AlignParams p{};
  p.E = E;
  p.bm = block_m;
  p.max_tiles = fmoe_max_tiles(n_slots, E);
  p.o.offs_raw = offs_raw;
  p.o.offs_pad = offs_pad;
  p.o.tile_map = tile_map;
  p.o.n_tiles = n_tiles;
  align_scan_kernel<<<1, kAlignThreads, 0, static_cast<hipStream_t>(stream)>>>(p, hist);
  return check_launch("expt_data");
}
