// C-ABI entry points of the GEMM stages and the whole fused path.
#include <cmath>
#include <mutex>

#include "gemm.hpp"

namespace fmoe {
int launch_prefill(WType wt, Mode mode, int bm, const GemmParams& p, hipStream_t s);
size_t prefill_tail_bytes(WType wt, int bm, int64_t max_tiles, int64_t Nout);
int decode_int4_row_split(int64_t max_tiles);
int launch_decode(WType wt, Mode mode, const GemmParams& p, hipStream_t s);
int launch_gemm1_token(const GemmParams& p, int E, int k, hipStream_t s);
int launch_gemm2_sum_token(const GemmParams& q, int E, int k, float scale, void* out, hipStream_t s);
int dequant_4bit(int wtype, const void* q, const void* scale, const void* zeros, int64_t E,
                 int64_t R, int64_t K, uint16_t* out, hipStream_t s);
int moe_sum_flat(const float* y, int splits, const int32_t* ids, int E, int64_t M, int k, int64_t K,
                 float scale, void* out, hipStream_t s);
int moe_sum_bf16(const uint16_t* y, const int32_t* gate_indx, int64_t M, int k, int64_t K,
                 float scale, void* out, hipStream_t s);
int launch_fused_int4(const GemmParams& p, const GemmParams& q, hipStream_t s);
bool fused_int4_fits(int64_t slots, int64_t K);
int moe_sum_planes(const float* y, int planes, const int32_t* gate_indx, const int32_t* ids, int E,
                   int64_t M, int k, int64_t K, float scale, void* out, hipStream_t s);
}  // namespace fmoe

using namespace fmoe;
using fmoe_host::fail;

namespace {

constexpr int kDecodeBM = 16;
constexpr int kDecodeBN = 64;
constexpr int kDecodeTargetWgs = 1024;
constexpr int kPrefillBN = 256;
constexpr int kPrefillTargetWgs = 6 * 256;
// at or above this many output tiles (2.5 waves of one workgroup per CU) the
// last wave's tail costs less than writing and re-reading fp32 split planes
// (reference sweep K=1280 N=3072 E=64 M=4096: 1.31 -> 1.19 ms unsplit)
constexpr int kPrefillNoSplitWgs = 640;

size_t al(size_t v) { return (v + 255) & ~size_t(255); }

bool valid_wtype(int wt) {
  return wt == FMOE_W_BF16 || wt == FMOE_W_FP8 || wt == FMOE_W_INT4 || wt == FMOE_W_MXFP4 ||
         wt == FMOE_W_INT4_TILED || wt == FMOE_W_MXFP4_TILED;
}
// weight formats that only the streaming (decode) kernels read
bool is_int4(int wt) { return wt == FMOE_W_INT4 || wt == FMOE_W_INT4_TILED; }
bool is_mx(int wt) { return wt == FMOE_W_MXFP4 || wt == FMOE_W_MXFP4_TILED; }
bool decode_only(int wt) { return is_int4(wt) || is_mx(wt); }
// 4-bit weights in the tiled layout of fmoe_tile_int4
bool is_tiled(int wt) { return wt == FMOE_W_INT4_TILED || wt == FMOE_W_MXFP4_TILED; }

WType to_wt(int wt) {
  return wt == FMOE_W_FP8 ? WType::kFp8
                          : (is_int4(wt) ? WType::kInt4 : (is_mx(wt) ? WType::kMxfp4 : WType::kBf16));
}

int check_routing(const fmoe_routing* r, const char* who) {
  if (!r) return fail(FMOE_ERR_INVALID, "%s: null routing", who);
  if (!r->topk_indx || !r->gate_scal || !r->offs_raw || !r->tile_map || !r->n_tiles)
    return fail(FMOE_ERR_INVALID, "%s: routing pointer is null", who);
  if (r->n_tokens < 0 || r->top_k < 1 || r->n_experts < 1 || r->max_tiles < 0)
    return fail(FMOE_ERR_INVALID, "%s: bad routing sizes", who);
  if (r->block_m != 16 && r->block_m != 64 && r->block_m != 128 && r->block_m != 160 &&
      r->block_m != 256)
    return fail(FMOE_ERR_UNSUPPORTED, "%s: block_m=%d is not supported", who, r->block_m);
  if (r->block_m != 16 && !r->offs_pad)
    return fail(FMOE_ERR_INVALID, "%s: prefill routing needs offs_pad", who);
  return FMOE_OK;
}

// Decode (block_m 16) or prefill (64 / 128) kernels follow the routing's tile height.
bool is_decode(const fmoe_routing* r) { return r->block_m == kDecodeBM; }

GemmParams base_params(const fmoe_routing* r) {
  GemmParams p{};
  p.topk_indx = r->topk_indx;
  p.gate_scal = r->gate_scal;
  p.offs_raw = r->offs_raw;
  p.offs_pad = r->offs_pad;
  p.tile_map = r->tile_map;
  p.n_tiles = r->n_tiles;
  p.top_k = r->top_k;
  p.n_experts = r->n_experts;
  p.max_tiles = r->max_tiles;
  p.splits = 1;
  p.act = FMOE_ACT_SILU;
  p.bias = nullptr;
  p.alpha = 1.0f;
  p.limit = 0.0f;
  return p;
}

// Tile height for the fused path: 16 = decode kernels, else the prefill tile,
// from the mean slots per expert (measured on the BASELINE shapes): bf16
// 256-row tiles once experts average >= 256 slots, 128-row tiles from 40
// (a half-empty 128-row tile still beats a 64-row one), else 64; 160-row
// tiles as below.
int choose_block_m(int wtype, int64_t M, int k, int E, int path) {
  const int64_t slots = M * k;
  const int64_t active = slots < E ? slots : E;
  if (decode_only(wtype) || path == 2) return kDecodeBM;
  if (path != 1 && slots <= kDecodeBM * (active > 0 ? active : 1)) return kDecodeBM;
  const int64_t mean = slots / E;
  if (wtype == FMOE_W_BF16 && mean >= 256) return 256;
  if (mean < 40) return 64;
  if (wtype == FMOE_W_FP8 || wtype == FMOE_W_BF16) {
    // 160-row tiles where they need fewer M-tiles per expert than 128-row
    // ones at the mean + 2 sd of a uniform routing's per-expert load (each
    // M-tile streams the expert's whole weight panel again)
    const double q = static_cast<double>(mean) + 2.0 * std::sqrt(static_cast<double>(mean));
    if (std::ceil(q / 160.0) < std::ceil(q / 128.0)) return 160;
  }
  return 128;
}

// The 160-row fp8 tile stages the weight scales of at most 64 reduction
// blocks (K, N <= 8192); larger fp8 layers take 128-row tiles.
int fit_block_m(int wtype, int bm, int64_t K, int64_t N) {
  return wtype == FMOE_W_FP8 && bm == 160 && (K > 8192 || N > 8192) ? 128 : bm;
}

}  // namespace

extern "C" int fmoe_choose_block_m(int wtype, int64_t M, int k, int E, int path) {
  return choose_block_m(wtype, M, k, E, path);
}

extern "C" int fmoe_fused_block_m(int wtype, int64_t M, int k, int E, int path, int64_t K, int64_t N) {
  return fit_block_m(wtype, choose_block_m(wtype, M, k, E, path), K, N);
}

extern "C" int fmoe_gemm2_splits(int wtype, int64_t K, int64_t N, const fmoe_routing* r, int path) {
  (void)path;
  if (!r) return 1;
  if (!is_decode(r)) {
    // Prefill GEMM2 has few output tiles (K / 256 per M-tile): below
    // kPrefillNoSplitWgs tiles, split the reduction dim until the grid covers
    // >= 6 waves of one workgroup per CU, so the last wave's tail stays small.
    // Partials are summed by moe_sum.
    const int64_t slots = r->n_tokens * r->top_k;
    const int64_t tiles = (slots + r->block_m - 1) / r->block_m;
    const int64_t wgs = tiles * ((K + kPrefillBN - 1) / kPrefillBN);
    if (wgs >= kPrefillNoSplitWgs) return 1;
    const int64_t stage_elems = wtype == FMOE_W_BF16 ? 32 : 128;
    int64_t sp = (kPrefillTargetWgs + wgs - 1) / (wgs > 0 ? wgs : 1);
    // each split keeps >= 64 stages: a short reduction gains less from the
    // split than its extra prologue / epilogue and fp32 planes cost (reference
    // sweep M=1024 / 2048, 48 stages: unsplit 549 -> 504 / 854 -> 738 us;
    // Mixtral M=4096, 224 stages, keeps its 3 splits)
    constexpr int64_t kMinStages = 64;
    const int64_t max_sp = N / stage_elems / kMinStages > 1 ? N / stage_elems / kMinStages : 1;
    if (sp > max_sp) sp = max_sp;
    if (sp > 4) sp = 4;
    return static_cast<int>(sp < 1 ? 1 : sp);
  }
  const int64_t slots = r->n_tokens * r->top_k;
  const int64_t est_tiles = slots < r->n_experts ? (slots > 0 ? slots : 1) : r->n_experts;
  // row workgroups: 64 rows each, or (row blocks) x 64 for the int4 row-split kernel
  const int rs = is_int4(wtype) ? decode_int4_row_split(r->max_tiles) : 0;
  const int64_t bn = rs > 0 ? rs * kDecodeBN : kDecodeBN;
  const int64_t ntiles = (K + bn - 1) / bn;
  const int64_t wgs = est_tiles * ntiles;
  const int64_t stage_elems = wtype == FMOE_W_BF16 ? 64 : 128;
  const int64_t nk = N / stage_elems;
  // as many splits as fit in the target without exceeding it (rounded down:
  // a grid already near the target runs better unsplit -- measured, e.g.
  // 896 base workgroups: 1 split 5% faster than 2)
  int64_t sp = kDecodeTargetWgs / wgs;
  const int64_t max_sp = nk / 4 > 1 ? nk / 4 : 1;  // keep >= 4 stages per split (one per wave)
  if (sp > max_sp) sp = max_sp;
  if (sp > 64) sp = 64;
  return static_cast<int>(sp < 1 ? 1 : sp);
}

extern "C" int fmoe_gemm1(int wtype, const void* x, const float* x_scale, const void* w13,
                          const void* w13_scale, const void* w13_zero, int64_t K, int64_t N,
                          const fmoe_routing* r, int gamma_on_input, void* act, int path,
                          void* stream) {
  return fmoe_gemm1_ex(wtype, x, x_scale, w13, w13_scale, w13_zero, K, N, r, gamma_on_input,
                       nullptr, act, path, stream);
}

namespace {
int check_epilogue(const fmoe_epilogue* ep, const char* who) {
  if (!ep) return FMOE_OK;
  if (ep->activation != FMOE_ACT_SILU && ep->activation != FMOE_ACT_GELU &&
      ep->activation != FMOE_ACT_SWIGLU)
    return fail(FMOE_ERR_INVALID, "%s: unknown activation %d", who, ep->activation);
  if (ep->bias && ep->activation != FMOE_ACT_SWIGLU)
    return fail(FMOE_ERR_UNSUPPORTED, "%s: bias with this activation is not supported", who);
  if (!(ep->alpha == ep->alpha) || !(ep->limit == ep->limit))
    return fail(FMOE_ERR_INVALID, "%s: alpha / limit must not be NaN", who);
  return FMOE_OK;
}
}  // namespace

namespace {
int gemm1_impl(int wtype, const void* x, const float* x_scale, const void* w13,
               const void* w13_scale, const void* w13_zero, int64_t K, int64_t N,
               const fmoe_routing* r, int gamma_on_input, const fmoe_epilogue* ep, void* act,
               int path, int4* tile_lut, uint8_t* act_q, float* act_qs, void* stream);
int gemm2_impl(int wtype, const void* act, const float* act_scale, const void* w2,
               const void* w2_scale, const void* w2_zero, int64_t K, int64_t N,
               const fmoe_routing* r, int apply_gamma, const float* bias, void* y, int splits,
               int path, int4* tile_lut, bool y_bf16, void* stream, float* tail_part = nullptr,
               size_t tail_bytes = 0);
}  // namespace

extern "C" int fmoe_gemm1_ex(int wtype, const void* x, const float* x_scale, const void* w13,
                             const void* w13_scale, const void* w13_zero, int64_t K, int64_t N,
                             const fmoe_routing* r, int gamma_on_input, const fmoe_epilogue* ep,
                             void* act, int path, void* stream) {
  return gemm1_impl(wtype, x, x_scale, w13, w13_scale, w13_zero, K, N, r, gamma_on_input, ep, act,
                    path, nullptr, nullptr, nullptr, stream);
}

namespace {
int gemm1_impl(int wtype, const void* x, const float* x_scale, const void* w13,
               const void* w13_scale, const void* w13_zero, int64_t K, int64_t N,
               const fmoe_routing* r, int gamma_on_input, const fmoe_epilogue* ep, void* act,
               int path, int4* tile_lut, uint8_t* act_q, float* act_qs, void* stream) {
  if (int st = check_epilogue(ep, "gemm1")) return st;
  if (int st = check_routing(r, "gemm1")) return st;
  if (!valid_wtype(wtype)) return fail(FMOE_ERR_INVALID, "gemm1: unknown weight type %d", wtype);
  // (the int4 kernels' per-stage scale / zero fetch assumes adjacent gate
  // and up rows are the split halves, not SWIGLU's interleaved pairs)
  if (is_int4(wtype) && ep && ep->activation == FMOE_ACT_SWIGLU)
    return fail(FMOE_ERR_UNSUPPORTED, "gemm1: int4 weights with SWIGLU are not supported");
  if (K <= 0 || N <= 0 || K % 128 != 0 || N % 128 != 0)
    return fail(FMOE_ERR_UNSUPPORTED, "gemm1: K=%lld N=%lld must be multiples of 128",
                static_cast<long long>(K), static_cast<long long>(N));
  if (!x || !w13 || (!act && !act_q)) return fail(FMOE_ERR_INVALID, "gemm1: null pointer");
  if (wtype == FMOE_W_FP8 && !w13_scale)
    return fail(FMOE_ERR_INVALID, "gemm1: fp8 needs w13_scale");
  if (wtype == FMOE_W_FP8 && !is_decode(r) && !x_scale)
    return fail(FMOE_ERR_INVALID, "gemm1: fp8 prefill needs pre-quantized x with x_scale");
  if (wtype == FMOE_W_FP8 && is_decode(r) && x_scale)
    return fail(FMOE_ERR_INVALID, "gemm1: fp8 decode takes bf16 x (quantized in-kernel); x_scale must be null");
  if (is_int4(wtype) && (!w13_scale || !w13_zero))
    return fail(FMOE_ERR_INVALID, "gemm1: int4 needs w13_scale and w13_zero");
  if (is_mx(wtype) && !w13_scale)
    return fail(FMOE_ERR_INVALID, "gemm1: mxfp4 needs w13_scale (e8m0 block scales)");
  if (decode_only(wtype) && !is_decode(r))
    return fail(FMOE_ERR_UNSUPPORTED, "gemm1: int4 / mxfp4 weights need block_m=16 routing");
  if ((path == 1 && is_decode(r)) || (path == 2 && !is_decode(r)))
    return fail(FMOE_ERR_INVALID, "gemm1: path %d does not match block_m=%d", path, r->block_m);
  GemmParams p = base_params(r);
  p.A = static_cast<const uint8_t*>(x);
  p.a_scale = x_scale;
  p.B = static_cast<const uint8_t*>(w13);
  p.b_scale = static_cast<const float*>(w13_scale);
  p.b_gscale = static_cast<const uint16_t*>(w13_scale);
  p.b_zero = static_cast<const uint8_t*>(w13_zero);
  p.b_mxscale = static_cast<const uint8_t*>(w13_scale);
  p.b_tiled = is_tiled(wtype);
  p.Kred = K;
  p.Nout = 2 * N;
  p.N_act = N;
  p.gamma = gamma_on_input;
  p.out = act;
  if (ep) {
    p.act = ep->activation;
    p.bias = ep->bias;
    p.alpha = ep->alpha;
    p.limit = ep->limit;
  }
  p.tile_lut = tile_lut;
  p.act_q = act_q;  // only the fp8 prefill kernels take it (the fused path checks)
  p.act_qs = act_qs;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (is_decode(r)) return launch_decode(to_wt(wtype), Mode::kGemm1Silu, p, s);
  return launch_prefill(to_wt(wtype), Mode::kGemm1Silu, r->block_m, p, s);
}
}  // namespace

extern "C" int fmoe_gemm2(int wtype, const void* act, const float* act_scale, const void* w2,
                          const void* w2_scale, const void* w2_zero, int64_t K, int64_t N,
                          const fmoe_routing* r, int apply_gamma, float* y, int splits, int path,
                          void* stream) {
  return fmoe_gemm2_ex(wtype, act, act_scale, w2, w2_scale, w2_zero, K, N, r, apply_gamma, nullptr,
                       y, splits, path, stream);
}

extern "C" int fmoe_gemm2_ex(int wtype, const void* act, const float* act_scale, const void* w2,
                             const void* w2_scale, const void* w2_zero, int64_t K, int64_t N,
                             const fmoe_routing* r, int apply_gamma, const float* bias, float* y,
                             int splits, int path, void* stream) {
  return gemm2_impl(wtype, act, act_scale, w2, w2_scale, w2_zero, K, N, r, apply_gamma, bias, y,
                    splits, path, nullptr, false, stream);
}

namespace {
int gemm2_impl(int wtype, const void* act, const float* act_scale, const void* w2,
               const void* w2_scale, const void* w2_zero, int64_t K, int64_t N,
               const fmoe_routing* r, int apply_gamma, const float* bias, void* y, int splits,
               int path, int4* tile_lut, bool y_bf16, void* stream, float* tail_part,
               size_t tail_bytes) {
  if (int st = check_routing(r, "gemm2")) return st;
  if (!valid_wtype(wtype)) return fail(FMOE_ERR_INVALID, "gemm2: unknown weight type %d", wtype);
  if (K <= 0 || N <= 0 || K % 128 != 0 || N % 128 != 0)
    return fail(FMOE_ERR_UNSUPPORTED, "gemm2: K=%lld N=%lld must be multiples of 128",
                static_cast<long long>(K), static_cast<long long>(N));
  if (!act || !w2 || !y) return fail(FMOE_ERR_INVALID, "gemm2: null pointer");
  if (wtype == FMOE_W_FP8 && !w2_scale)
    return fail(FMOE_ERR_INVALID, "gemm2: fp8 needs w2_scale");
  if (wtype == FMOE_W_FP8 && !is_decode(r) && !act_scale)
    return fail(FMOE_ERR_INVALID, "gemm2: fp8 prefill needs pre-quantized act with act_scale");
  if (wtype == FMOE_W_FP8 && is_decode(r) && act_scale)
    return fail(FMOE_ERR_INVALID, "gemm2: fp8 decode takes bf16 act (quantized in-kernel); act_scale must be null");
  if (is_int4(wtype) && (!w2_scale || !w2_zero))
    return fail(FMOE_ERR_INVALID, "gemm2: int4 needs w2_scale and w2_zero");
  if (is_mx(wtype) && !w2_scale)
    return fail(FMOE_ERR_INVALID, "gemm2: mxfp4 needs w2_scale (e8m0 block scales)");
  if (decode_only(wtype) && !is_decode(r))
    return fail(FMOE_ERR_UNSUPPORTED, "gemm2: int4 / mxfp4 weights need block_m=16 routing");
  if ((path == 1 && is_decode(r)) || (path == 2 && !is_decode(r)))
    return fail(FMOE_ERR_INVALID, "gemm2: path %d does not match block_m=%d", path, r->block_m);
  if (splits < 1 || splits > 64)
    return fail(FMOE_ERR_INVALID, "gemm2: splits=%d out of range", splits);
  GemmParams p = base_params(r);
  p.A = static_cast<const uint8_t*>(act);
  p.a_scale = act_scale;
  p.B = static_cast<const uint8_t*>(w2);
  p.b_scale = static_cast<const float*>(w2_scale);
  p.b_gscale = static_cast<const uint16_t*>(w2_scale);
  p.b_zero = static_cast<const uint8_t*>(w2_zero);
  p.b_mxscale = static_cast<const uint8_t*>(w2_scale);
  p.b_tiled = is_tiled(wtype);
  p.Kred = N;
  p.Nout = K;
  p.N_act = N;
  p.gamma = apply_gamma;
  p.bias = bias;
  p.out = y;
  p.y_bf16 = y_bf16 && !is_decode(r) && splits == 1;
  p.splits = splits;
  p.out_split_stride = r->n_tokens * r->top_k * K;
  p.tile_lut = tile_lut;
  // fused prefill: tail split instead of split-K planes (the launcher turns
  // it off when the buffer or the runtime's occupancy query falls short)
  p.tail_split = (tail_part && !is_decode(r) && p.y_bf16) ? kTailMaxSplit : 0;
  p.tail_part = tail_part;
  p.tail_bytes = tail_bytes;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (is_decode(r)) return launch_decode(to_wt(wtype), Mode::kGemm2, p, s);
  return launch_prefill(to_wt(wtype), Mode::kGemm2, r->block_m, p, s);
}
}  // namespace

// ------------------------------------------------------------ fused path
namespace {

struct FusedLayout {
  int bm;
  int splits;
  bool y_bf16;
  bool fused4;  // one-launch int4 decode (splits = N / 128 planes)
  int64_t max_tiles;
  size_t align_ws, expt_indx, expt_scal, topk_indx, gate_indx, gate_scal, hist, offs_raw,
      offs_pad, tile_map, n_tiles, xq, xs, act, actq, acts, y, lut, tail, total;
  size_t tail_bytes;  // prefill GEMM2 tail-split partials (0: split-K planes or none)
};

int check_fused(const fmoe_fused_args* a) {
  if (!a) return fail(FMOE_ERR_INVALID, "fused_experts: null args");
  if (!valid_wtype(a->wtype)) return fail(FMOE_ERR_INVALID, "fused_experts: unknown weight type");
  if (a->M < 0 || a->E < 1 || a->E > 1024 || a->top_k < 1 || a->top_k > 32 || a->top_k > a->E)
    return fail(FMOE_ERR_INVALID, "fused_experts: bad M/E/top_k");
  if (a->K <= 0 || a->N <= 0 || a->K % 128 != 0 || a->N % 128 != 0)
    return fail(FMOE_ERR_UNSUPPORTED, "fused_experts: K=%lld N=%lld must be multiples of 128",
                static_cast<long long>(a->K), static_cast<long long>(a->N));
  if (is_int4(a->wtype) && a->activation == FMOE_ACT_SWIGLU)
    return fail(FMOE_ERR_UNSUPPORTED, "fused_experts: int4 weights with SWIGLU are not supported");
  if (is_int4(a->wtype) && a->group_size != 128)
    return fail(FMOE_ERR_UNSUPPORTED, "fused_experts: int4 group_size=%d is not supported",
                a->group_size);
  if (a->path < 0 || a->path > 2) return fail(FMOE_ERR_INVALID, "fused_experts: path %d", a->path);
  fmoe_epilogue ep{a->activation, a->b13, a->alpha, a->limit};
  if (int st = check_epilogue(&ep, "fused_experts")) return st;
  return FMOE_OK;
}

// Tiled int4 decode of the smallest batches runs as one launch per call
// (fused_int4_kernel: GEMM1, activation and GEMM2 of a 128-column slice of
// the intermediate per workgroup) plus the plane sum.  Its N / 128 fp32
// partial planes per slot grow with M, so larger batches keep the two GEMM
// launches.
// (The kernel applies no bias; calls with b13 / b2 take the two-launch route.)
constexpr int64_t kFusedInt4MaxM = 1;
bool fused_int4_route(const fmoe_fused_args* a, int bm) {
  return a->wtype == FMOE_W_INT4_TILED && bm == kDecodeBM && a->activation != FMOE_ACT_SWIGLU &&
         !a->b13 && !a->b2 && a->M <= kFusedInt4MaxM && a->top_k <= 32 &&
         fused_int4_fits(a->M * a->top_k, a->K);
}

FusedLayout layout(const fmoe_fused_args* a) {
  FusedLayout L{};
  const int64_t slots = a->M * a->top_k;
  L.bm = fit_block_m(a->wtype, choose_block_m(a->wtype, a->M, a->top_k, a->E, a->path), a->K, a->N);
  L.max_tiles = fmoe_max_tiles(slots, a->E);
  fmoe_routing r{};
  r.n_tokens = a->M;
  r.top_k = a->top_k;
  r.n_experts = a->E;
  r.block_m = L.bm;
  r.max_tiles = static_cast<int32_t>(L.max_tiles);
  L.fused4 = fused_int4_route(a, L.bm);
  L.splits = L.fused4 ? static_cast<int>(a->N / 128) : fmoe_gemm2_splits(a->wtype, a->K, a->N, &r, 0);
  // Prefill GEMM2 that the split rule would cut into fp32 planes (few tiles,
  // a long reduction): whole tiles store bf16 rows instead and only the
  // tiles of each XCD's last partial round are split (tail_fold_kernel adds
  // their partials).  Mixtral M=4096: GEMM2 + sum 1027 -> 917 us.  Where the
  // rule keeps whole tiles, splitting the last round lost (the split
  // workgroups' prologue, fp32 stores and fold cost more than the idle
  // slots: Qwen3 M=8192 GEMM2 351 -> 387 us, DSV3 M=4096 1107 -> 1158 us).
  L.tail_bytes = (L.bm != kDecodeBM && !L.fused4 && L.splits > 1 &&
                  (a->wtype == FMOE_W_BF16 || a->wtype == FMOE_W_FP8))
                     ? prefill_tail_bytes(to_wt(a->wtype), L.bm, L.max_tiles, a->K)
                     : 0;
  if (L.tail_bytes > 0) L.splits = 1;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += al(bytes);
    return o;
  };
  L.align_ws = take(fmoe_align_workspace_bytes(a->M, a->top_k, a->E));
  L.expt_indx = take(4 * slots);
  L.expt_scal = take(4 * slots);
  L.topk_indx = take(4 * slots);
  L.gate_indx = take(4 * slots);
  L.gate_scal = take(4 * slots);
  L.hist = take(4 * a->E);
  L.offs_raw = take(4 * (a->E + 1));
  L.offs_pad = take(4 * (a->E + 1));
  L.tile_map = take(4 * L.max_tiles);
  L.n_tiles = take(4);
  const bool fp8 = a->wtype == FMOE_W_FP8 && L.bm != kDecodeBM;
  L.xq = take(fp8 ? a->M * a->K : 0);
  L.xs = take(fp8 ? 4 * a->M * (a->K / 128) : 0);
  L.act = take(fp8 ? 0 : 2 * slots * a->N);  // fp8 prefill: GEMM1 writes the quantized act
  L.actq = take(fp8 ? slots * a->N : 0);
  L.acts = take(fp8 ? 4 * slots * (a->N / 128) : 0);
  // prefill with one split: bf16 rows (see fused path); otherwise fp32 planes
  L.y_bf16 = L.bm != kDecodeBM && L.splits == 1;
  L.y = take((L.y_bf16 ? 2 : 4) * static_cast<size_t>(L.splits) * slots * a->K);
  // prefill: logical-tile table, shared by the two GEMM launches (stream order)
  const int64_t nn1 = (a->N + kPrefillBN / 2 - 1) / (kPrefillBN / 2);
  const int64_t nn2 = (a->K + kPrefillBN - 1) / kPrefillBN;
  L.lut = take(L.bm == kDecodeBM ? 0 : 16 * static_cast<size_t>(L.max_tiles) * (nn1 > nn2 ? nn1 : nn2));
  L.tail = take(L.tail_bytes);
  L.total = off;
  return L;
}

// Tiny decode batches: every tile holds at most 16 slots and the whole
// routing fits one workgroup's LDS, so the GEMM workgroups compute their own
// tile from the top-k ids (no align launch); rows are flat slots t * k + j.
// bf16 / fp8 up to 16 tokens; int4 only for a single token (Mixtral shape:
// M = 1 60.8 -> 58.5 us, M = 4 / 16 slower than with the align launch, whose
// tiles let the GEMM workgroups start without the routing latency); MXFP4
// never (measured slower).
bool tiny_decode(const fmoe_fused_args* a, const FusedLayout& L) {
  const int64_t max_m = is_int4(a->wtype) ? 1 : (is_mx(a->wtype) ? 0 : 16);
  return L.bm == kDecodeBM && a->M <= max_m && a->M * a->top_k <= 512 && a->E <= 1024 &&
         !a->expert_map;
}

// GEMM1 / GEMM2 parameters of the fused decode path; g1 comes in with the
// routing fields set (tile map or tiny-batch ids), g2 starts as its copy.
void decode_pair(const fmoe_fused_args* a, const FusedLayout& L, char* ws, GemmParams& g1, GemmParams& g2) {
  g1.splits = 1;
  g1.alpha = a->alpha;
  g1.limit = a->limit;
  g1.act = a->activation;
  g2 = g1;
  g1.A = static_cast<const uint8_t*>(a->x);
  g1.B = static_cast<const uint8_t*>(a->w13);
  g1.b_scale = static_cast<const float*>(a->w13_scale);
  g1.b_gscale = static_cast<const uint16_t*>(a->w13_scale);
  g1.b_zero = static_cast<const uint8_t*>(a->w13_zero);
  g1.b_mxscale = static_cast<const uint8_t*>(a->w13_scale);
  g1.b_tiled = is_tiled(a->wtype);
  g1.Kred = a->K;
  g1.Nout = 2 * a->N;
  g1.N_act = a->N;
  g1.gamma = a->apply_router_weight_on_input;
  g1.bias = a->b13;
  g1.out = ws + L.act;
  g2.act = FMOE_ACT_SILU;
  g2.A = static_cast<const uint8_t*>(g1.out);
  g2.B = static_cast<const uint8_t*>(a->w2);
  g2.b_scale = static_cast<const float*>(a->w2_scale);
  g2.b_gscale = static_cast<const uint16_t*>(a->w2_scale);
  g2.b_zero = static_cast<const uint8_t*>(a->w2_zero);
  g2.b_mxscale = static_cast<const uint8_t*>(a->w2_scale);
  g2.b_tiled = is_tiled(a->wtype);
  g2.Kred = a->N;
  g2.Nout = a->K;
  g2.N_act = a->N;
  g2.gamma = !a->apply_router_weight_on_input;
  g2.bias = a->b2;
  g2.out = ws + L.y;
  g2.splits = L.splits;
  g2.out_split_stride = a->M * a->top_k * a->K;
}

int fused_tiny(const fmoe_fused_args* a, const FusedLayout& L, char* ws, hipStream_t s) {
  const int64_t slots = a->M * a->top_k;
  GemmParams g1{}, g2;
  g1.top_k = a->top_k;
  g1.n_experts = a->E;
  g1.max_tiles = static_cast<int>(fmoe_max_tiles(slots, a->E));
  g1.tiny_ids = a->topk_ids;
  g1.tiny_w = a->topk_weights;
  g1.n_tokens = a->M;
  decode_pair(a, L, ws, g1, g2);
  const float* y = reinterpret_cast<const float*>(ws + L.y);
  if (L.fused4) {
    if (int st = launch_fused_int4(g1, g2, s)) return st;
    return moe_sum_planes(y, L.splits, nullptr, a->topk_ids, a->E, a->M, a->top_k, a->K,
                          a->routed_scaling_factor, a->out, s);
  }
  // one bf16 token: GEMM1 as a row-parallel dot (more workgroups than 64-row blocks)
  if (a->M == 1 && a->wtype == FMOE_W_BF16) {
    if (int st = launch_gemm1_token(g1, a->E, a->top_k, s)) return st;
  } else if (int st = launch_decode(to_wt(a->wtype), Mode::kGemm1Silu, g1, s)) {
    return st;
  }
  // one bf16 token: GEMM2 and the top-k sum in one launch
  if (a->M == 1 && a->wtype == FMOE_W_BF16 && a->M * a->top_k <= 32)
    return launch_gemm2_sum_token(g2, a->E, a->top_k, a->routed_scaling_factor, a->out, s);
  if (int st = launch_decode(to_wt(a->wtype), Mode::kGemm2, g2, s)) return st;
  return moe_sum_flat(y, L.splits, a->topk_ids, a->E, a->M, a->top_k, a->K, a->routed_scaling_factor,
                      a->out, s);
}

}  // namespace

// Large batches of 4-bit weights: the decode kernels re-read an expert's
// weights for every 16-slot tile, so once experts average kDequantMinSlots
// slots the weights are dequantized once to bf16 (in the workspace) and the
// bf16 prefill kernels run on them.  Measured on the Mixtral shape (tiled
// int4, decode kernels vs dequantize + bf16 prefill): M=512 (128 slots per
// expert) 1.16 vs 1.66 ms, M=1024 (256) 2.20 vs 2.13 ms, M=4096 8.4 vs 3.8 ms;
// MXFP4 M=1024 2.81 vs 2.14 ms.
constexpr int64_t kDequantMinSlots = 256;

// The bf16 copies live in the caller's workspace for the duration of the
// call (2 * E * 3 * N * K bytes: 2.8 GB for the Mixtral shape), so the route is
// taken automatically only while they stay within kDequantMaxBytes; above it
// (e.g. a DeepSeek-size int4 layer, ~22 GB) the decode kernels run at every M.
// path = 1 asks for the route regardless of the size.
constexpr size_t kDequantMaxBytes = size_t(4) << 30;

// bytes of the bf16 copies of w13 and w2
size_t dequant_bytes(const fmoe_fused_args* a) {
  return al(2 * static_cast<size_t>(a->E) * 2 * a->N * a->K) + al(2 * static_cast<size_t>(a->E) * a->K * a->N);
}

bool dequant_prefill(const fmoe_fused_args* a) {
  if (!decode_only(a->wtype) || a->path == 2) return false;
  if (a->path == 1) return true;
  return a->M * a->top_k >= kDequantMinSlots * a->E && dequant_bytes(a) <= kDequantMaxBytes;
}

// The same call on bf16 copies of the weights placed at the workspace start.
fmoe_fused_args bf16_args(const fmoe_fused_args* a, void* ws) {
  fmoe_fused_args b = *a;
  b.wtype = FMOE_W_BF16;
  b.w13_scale = b.w2_scale = nullptr;
  b.w13_zero = b.w2_zero = nullptr;
  b.path = 1;
  b.w13 = b.w2 = nullptr;  // size queries only
  if (ws) {
    b.w13 = ws;
    b.w2 = static_cast<char*>(ws) + al(2 * static_cast<size_t>(a->E) * 2 * a->N * a->K);
    b.workspace = static_cast<char*>(ws) + dequant_bytes(a);
    b.workspace_bytes = a->workspace_bytes - dequant_bytes(a);
  }
  return b;
}

extern "C" size_t fmoe_fused_experts_workspace_bytes(const fmoe_fused_args* a) {
  if (check_fused(a) != FMOE_OK) return 0;
  if (dequant_prefill(a)) {
    const fmoe_fused_args b = bf16_args(a, nullptr);
    return dequant_bytes(a) + layout(&b).total;
  }
  return layout(a).total;
}

extern "C" int fmoe_fused_experts(const fmoe_fused_args* a, void* stream) {
  if (int st = check_fused(a)) return st;
  if (a->M == 0) return FMOE_OK;
  if (!a->x || !a->w13 || !a->w2 || !a->topk_ids || !a->topk_weights || !a->out)
    return fail(FMOE_ERR_INVALID, "fused_experts: null pointer");
  if (dequant_prefill(a)) {
    const size_t need = fmoe_fused_experts_workspace_bytes(a);
    if (!a->workspace || a->workspace_bytes < need)
      return fail(FMOE_ERR_WORKSPACE, "fused_experts: workspace %zu < %zu bytes", a->workspace_bytes, need);
    const fmoe_fused_args b = bf16_args(a, a->workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int st = dequant_4bit(a->wtype, a->w13, a->w13_scale, a->w13_zero, a->E, 2 * a->N, a->K,
                              static_cast<uint16_t*>(const_cast<void*>(b.w13)), s))
      return st;
    if (int st = dequant_4bit(a->wtype, a->w2, a->w2_scale, a->w2_zero, a->E, a->K, a->N,
                              static_cast<uint16_t*>(const_cast<void*>(b.w2)), s))
      return st;
    return fmoe_fused_experts(&b, stream);
  }
  const FusedLayout L = layout(a);
  if (!a->workspace || a->workspace_bytes < L.total)
    return fail(FMOE_ERR_WORKSPACE, "fused_experts: workspace %zu < %zu bytes", a->workspace_bytes,
                L.total);
  char* ws = static_cast<char*>(a->workspace);
  auto at = [&](size_t o) { return static_cast<void*>(ws + o); };
  if (tiny_decode(a, L)) return fused_tiny(a, L, ws, static_cast<hipStream_t>(stream));

  fmoe_align_out o{};
  o.expt_indx = static_cast<int32_t*>(at(L.expt_indx));
  o.expt_scal = static_cast<float*>(at(L.expt_scal));
  o.topk_indx = static_cast<int32_t*>(at(L.topk_indx));
  o.gate_indx = static_cast<int32_t*>(at(L.gate_indx));
  o.gate_scal = static_cast<float*>(at(L.gate_scal));
  o.hist = static_cast<int32_t*>(at(L.hist));
  o.offs_raw = static_cast<int32_t*>(at(L.offs_raw));
  o.offs_pad = static_cast<int32_t*>(at(L.offs_pad));
  o.tile_map = static_cast<int32_t*>(at(L.tile_map));
  o.n_tiles = static_cast<int32_t*>(at(L.n_tiles));
  if (int st = fmoe_align_ex(a->topk_ids, a->topk_weights, a->M, a->top_k, a->E, L.bm,
                             a->expert_map, a->n_global, &o, at(L.align_ws),
                             fmoe_align_workspace_bytes(a->M, a->top_k, a->E), stream))
    return st;

  fmoe_routing r{};
  r.topk_indx = o.topk_indx;
  r.gate_indx = o.gate_indx;
  r.gate_scal = o.gate_scal;
  r.offs_raw = o.offs_raw;
  r.offs_pad = o.offs_pad;
  r.tile_map = o.tile_map;
  r.n_tiles = o.n_tiles;
  r.n_tokens = a->M;
  r.top_k = a->top_k;
  r.n_experts = a->E;
  r.block_m = L.bm;
  r.max_tiles = static_cast<int32_t>(L.max_tiles);

  // fp8 prefill quantizes activations in separate passes; the decode kernels
  // quantize their bf16 rows in registers
  const bool fp8 = a->wtype == FMOE_W_FP8 && L.bm != kDecodeBM;
  const void* x = a->x;
  const float* xs = nullptr;
  if (fp8) {
    if (int st = fmoe_quant_fp8_group(a->x, a->M, a->K, 128, at(L.xq),
                                      static_cast<float*>(at(L.xs)), stream))
      return st;
    x = at(L.xq);
    xs = static_cast<const float*>(at(L.xs));
  }
  if (L.fused4) {
    GemmParams g1 = base_params(&r), g2;
    decode_pair(a, L, ws, g1, g2);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int st = launch_fused_int4(g1, g2, s)) return st;
    return moe_sum_planes(static_cast<const float*>(at(L.y)), L.splits, o.gate_indx, nullptr, a->E, a->M,
                          a->top_k, a->K, a->routed_scaling_factor, a->out, s);
  }
  fmoe_epilogue ep{a->activation, a->b13, a->alpha, a->limit};
  int4* lut = L.bm == kDecodeBM ? nullptr : static_cast<int4*>(at(L.lut));
  // fp8 prefill: the GEMM1 epilogue quantizes the activation (1x128 groups,
  // bit-identical to fmoe_quant_fp8_group on its bf16 rows)
  uint8_t* actq = fp8 ? static_cast<uint8_t*>(at(L.actq)) : nullptr;
  float* actqs = fp8 ? static_cast<float*>(at(L.acts)) : nullptr;
  if (int st = gemm1_impl(a->wtype, x, xs, a->w13, a->w13_scale, a->w13_zero, a->K, a->N, &r,
                          a->apply_router_weight_on_input, &ep, fp8 ? nullptr : at(L.act), 0, lut,
                          actq, actqs, stream))
    return st;
  const void* act = fp8 ? static_cast<const void*>(actq) : at(L.act);
  const float* acts = actqs;
  // Prefill without split-K keeps each slot's GEMM2 row in bf16 until the
  // top-k sum (SGLang's per-slot intermediate has the same rounding point);
  // split-K planes and the decode path stay fp32.
  if (int st = gemm2_impl(a->wtype, act, acts, a->w2, a->w2_scale, a->w2_zero, a->K, a->N, &r,
                          !a->apply_router_weight_on_input, a->b2, at(L.y), L.splits, 0, lut,
                          L.y_bf16, stream, L.tail_bytes ? static_cast<float*>(at(L.tail)) : nullptr,
                          L.tail_bytes))
    return st;
  if (L.y_bf16)
    return moe_sum_bf16(static_cast<const uint16_t*>(at(L.y)), o.gate_indx, a->M, a->top_k, a->K,
                        a->routed_scaling_factor, a->out, static_cast<hipStream_t>(stream));
  return fmoe_moe_sum(static_cast<const float*>(at(L.y)), L.splits, o.gate_indx, a->M, a->top_k,
                      a->K, a->routed_scaling_factor, a->out, stream);
}

// ------------------------------------------------ no-allocation entry point
namespace fmoe {
// The workspace of fmoe_fused_experts_noalloc: one copy per GPU, in the code
// object's device memory.  Host code never uses this name as an address (it
// is a host-side stand-in): the device address comes from
// hipGetSymbolAddress, once per device.
__device__ __align__(256) char scratch[FMOE_NOALLOC_SCRATCH_BYTES];
}  // namespace fmoe

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices];

// Device address of the current device's scratch array (looked up on the
// first call on that device).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FMOE_ERR_HIP, "fused_experts_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FMOE_ERR_UNSUPPORTED, "fused_experts_noalloc: device %d is not supported", dev);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(fmoe::scratch));
    if (e != hipSuccess || !p)
      return fail(FMOE_ERR_HIP, "fused_experts_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return FMOE_OK;
}
}  // namespace

extern "C" int fmoe_fused_experts_noalloc(const fmoe_fused_args* a, void* stream) {
  if (int st = check_fused(a)) return st;
  const size_t need = fmoe_fused_experts_workspace_bytes(a);
  if (need > FMOE_NOALLOC_SCRATCH_BYTES)
    return fail(FMOE_ERR_UNSUPPORTED,
                "fused_experts_noalloc: this call needs %zu bytes of workspace, above the %zu-byte "
                "scratch maximum (use fmoe_fused_experts with a caller workspace)",
                need, static_cast<size_t>(FMOE_NOALLOC_SCRATCH_BYTES));
  void* ws = nullptr;
  if (int st = scratch_for_current_device(&ws)) return st;
  fmoe_fused_args b = *a;
  b.workspace = ws;
  b.workspace_bytes = FMOE_NOALLOC_SCRATCH_BYTES;
  return fmoe_fused_experts(&b, stream);
}
