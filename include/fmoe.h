/*
 * fmoe.h — C ABI of the MI355X (gfx950) fused-MoE library `libfmoe.so`.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream passed
 * as `void*` (a hipStream_t; NULL = the default stream), enqueues its kernels
 * on that stream and returns a status code without synchronising.  Nothing
 * here allocates device memory: buffers, including workspaces whose size the
 * matching *_bytes() query reports, belong to the caller.  Calls are
 * re-entrant; concurrent calls must not share output or workspace buffers.
 *
 * Reference interfaces each entry replaces are cited as path:line relative to
 * the FlagGems-sglang source root (src/flaggems_sglang/...).
 *
 * Tensor layouts (row-major, contiguous):
 *   hidden states x      [M, K]          bf16 (fp8 path: quantized in-library)
 *   w13 (gate ; up)      [E, 2N, K]      bf16 | fp8-e4m3fn | uint4 packed [E, 2N, K/2]
 *   w2                   [E, K, N]       bf16 | fp8-e4m3fn | uint4 packed [E, K, N/2]
 *   fp8 weight scales    w13 [E, 2N/128, K/128], w2 [E, K/128, N/128]   fp32
 *   int4 scales          w13 [E, K/g, 2N] fp16, w2 [E, N/g, K] fp16    (group g)
 *   int4 zeros           w13 [E, K/g, N]  u8 (2 per byte), w2 [E, N/g, K/2] u8
 *   topk_ids/topk_weights [M, k]         int32 / fp32
 *   output               [M, K]          bf16
 * "slots" are the M*k (token, expert) pairs; the routing below orders them by
 * expert (stable: ascending token within an expert).
 */
#ifndef FMOE_H_
#define FMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status codes */
enum fmoe_status {
  FMOE_OK = 0,
  FMOE_ERR_INVALID = 1,     /* bad pointer / shape / value (reference: assert) */
  FMOE_ERR_UNSUPPORTED = 2, /* feature or shape not implemented ("... is not supported") */
  FMOE_ERR_WORKSPACE = 3,   /* workspace smaller than the *_bytes() query */
  FMOE_ERR_HIP = 4,         /* a HIP runtime / launch error */
};

enum fmoe_wtype {
  FMOE_W_BF16 = 0,     /* bf16 weights, bf16 activations */
  FMOE_W_FP8 = 1,      /* fp8 e4m3fn weights with 128x128 block scales, 1x128 dynamic activation quant */
  FMOE_W_INT4 = 2,     /* uint4 weights with fp16 group scales and uint4 zeros, bf16 activations */
  FMOE_W_MXFP4 = 3,    /* OCP MXFP4 weights (e2m1, one e8m0 scale per 32 along the reduction
                          dim), bf16 activations: w13 [E, 2N, K/2] u8 + scale [E, 2N, K/32] u8,
                          w2 [E, K, N/2] u8 + scale [E, K, N/32] u8; element 2i in the low
                          nibble; w = e2m1(q) * 2^(s - 127) */
  FMOE_W_INT4_TILED = 4, /* FMOE_W_INT4 with the weight bytes tiled for the decode kernels
                            (scales and zeros unchanged): w13 [E, 2N/16, K/128, 1024],
                            w2 [E, K/16, N/128, 1024]; see fmoe_tile_int4 */
  FMOE_W_MXFP4_TILED = 5, /* FMOE_W_MXFP4 with the weight bytes tiled the same way
                             (fmoe_tile_int4; e8m0 scales unchanged) */
};

/* GEMM1 activations (the fused epilogue of fmoe_gemm1_ex / fmoe_fused_experts). */
enum fmoe_activation {
  FMOE_ACT_SILU = 0,   /* silu(gate) * up, gate rows 0..N-1, up rows N..2N-1 (ops/fused_moe.py:28-47) */
  FMOE_ACT_GELU = 1,   /* gelu(gate) * up with the exact (erf) GELU, same split (ops/fused_moe.py:203-204) */
  FMOE_ACT_SWIGLU = 2, /* swiglu of the bias path (ops/fused_moe.py:258-259): rows interleaved,
                          gate = row 2j, linear = row 2j+1; see fmoe_epilogue.  Not with int4
                          weights (FMOE_ERR_UNSUPPORTED) */
};

/* Text of a status code, and the message of the last failure on this thread. */
const char* fmoe_status_string(int status);
const char* fmoe_last_error(void);
int fmoe_abi_version(void);

/* --------------------------------------------------------------- routing
 * Router: logits [M, E] fp32 -> topk_weights [M, k] fp32, topk_ids [M, k]
 * int32, in descending score order.
 *
 * fmoe_topk_softmax replaces the softmax -> torch.topk -> renormalise
 * sequence of tests/test_fused_moe.py:24-27 (SGLang's fused_topk).
 * Requires 1 <= k <= 32, k <= E <= 1024.
 */
int fmoe_topk_softmax(const float* logits, int64_t M, int E, int k, int renormalize,
                      float* topk_weights, int32_t* topk_ids, void* stream);

/* Grouped top-k (DeepSeek-V3 routing; SGLang biased_grouped_topk, external to
 * the reference): scores = sigmoid(logits) (scoring 0) or softmax (1);
 * selection on scores + bias (bias may be NULL); group score = sum of top-2
 * in each of n_group groups; the topk_group best groups are kept; k experts
 * picked by biased score; weights are the unbiased scores, renormalised.
 * Requires E % n_group == 0, E / n_group >= 2, E <= 1024, n_group <= 64. */
int fmoe_grouped_topk(const float* logits, const float* bias, int64_t M, int E, int k,
                      int n_group, int topk_group, int scoring, int renormalize,
                      float* topk_weights, int32_t* topk_ids, void* stream);

/* ------------------------------------------------------------- alignment
 * Replaces _standard_topk_to_triton_kernels (ops/fused_moe.py:103-130) plus
 * triton_kernels.routing.compute_expt_data_torch (called at :124) and
 * SGLang's moe_align_block_size, in one deterministic pass (histogram ->
 * exclusive scan -> stable scatter).  Outputs (device, caller-allocated):
 *
 *   expt_indx   [M*k]  int32  per-token ascending expert ids, flattened (:114-117)
 *   expt_scal   [M*k]  fp32   weights gathered alongside (:115-116)
 *   topk_indx   [M*k]  int32  expert-sorted slot -> flat index (:118)
 *   gate_indx   [M*k]  int32  inverse permutation (:119)
 *   gate_scal   [M*k]  fp32   weight of each sorted slot (:120)
 *   hist        [E]    int32  slots per expert (:121-123)
 *   offs_raw    [E+1]  int32  ExptData.token_offs_raw
 *   offs_pad    [E+1]  int32  ExptData.token_offs_pad[block_m] (in tiles)
 *   tile_map    [fmoe_max_tiles()] int32  ExptData.block_pid_map[block_m]:
 *                              (tile_in_expert << 16) | expert, -1 unused
 *   n_tiles     [1]    int32  used tiles
 *   sorted_token_ids [fmoe_sorted_ids_len()] int32 (may be NULL): SGLang
 *              moe_align_block_size format, flat indices of topk_ids, padded
 *              per expert to block_m with the sentinel M*k
 *   expert_ids [fmoe_sorted_ids_len()/block_m + 1] int32 (may be NULL): expert
 *              of each block_m block, -1 past the used blocks
 *   num_tokens_post_padded [1] int32 (may be NULL)
 *
 * topk_ids values must lie in [0, E) and be distinct within a row;
 * FMOE_ERR_INVALID is not detectable for out-of-range ids without a device
 * sync, so ids >= E are counted into no expert and their slots are dropped
 * (gate_scal 0, never read by the GEMMs).
 * Requires 1 <= k <= 32, 1 <= E <= 1024, block_m in {16, 32, 64, 128}.
 */
typedef struct fmoe_align_out {
  int32_t* expt_indx;
  float* expt_scal;
  int32_t* topk_indx;
  int32_t* gate_indx;
  float* gate_scal;
  int32_t* hist;
  int32_t* offs_raw;
  int32_t* offs_pad;
  int32_t* tile_map;
  int32_t* n_tiles;
  int32_t* sorted_token_ids;
  int32_t* expert_ids;
  int32_t* num_tokens_post_padded;
} fmoe_align_out;

int64_t fmoe_max_tiles(int64_t n_slots, int E);
int64_t fmoe_sorted_ids_len(int64_t n_slots, int E, int block_m);
size_t fmoe_align_workspace_bytes(int64_t M, int k, int E);
int fmoe_align(const int32_t* topk_ids, const float* topk_weights, int64_t M, int k, int E,
               int block_m, const fmoe_align_out* out, void* workspace, size_t workspace_bytes,
               void* stream);

/* ExptData from a histogram alone (compute_expt_data_torch; used when the
 * caller already holds triton_kernels-format routing, ops/fused_moe.py:339-340). */
/* fmoe_align with an expert map (expert parallel; the reference's
 * expert_map / global_num_experts arguments, ops/fused_moe.py:145-146,160):
 * topk_ids hold global ids in [0, n_global); expert_map [n_global] int32 maps
 * each to a local expert in [0, E) or to -1.  Slots whose expert is not local
 * are dropped (gate_indx = -1, no GEMM rows; their tokens get contributions
 * from the local experts only).  expert_map null = identity (fmoe_align). */
int fmoe_align_ex(const int32_t* topk_ids, const float* topk_weights, int64_t M, int k, int E,
                  int block_m, const int32_t* expert_map, int n_global,
                  const fmoe_align_out* out, void* workspace, size_t workspace_bytes,
                  void* stream);

int fmoe_expt_data(const int32_t* hist, int E, int64_t n_slots, int block_m, int32_t* offs_raw,
                   int32_t* offs_pad, int32_t* tile_map, int32_t* n_tiles, void* stream);

/* ------------------------------------------------------------ quantization
 * Dynamic per-token-group fp8 quant (SGLang per_token_group_quant_fp8):
 * scale = max(amax, 1e-10) / 448, q = e4m3fn(clamp(x / scale, +-448)) (RNE).
 * x [M, K] bf16 -> q [M, K] fp8, scale [M, K/group] fp32.  K % group == 0,
 * group in {64, 128}. */
int fmoe_quant_fp8_group(const void* x, int64_t M, int64_t K, int group, void* q, float* scale,
                         void* stream);

/* ------------------------------------------------------------------- GEMMs
 * Routing view the GEMMs read (all device pointers from fmoe_align /
 * fmoe_expt_data for the same block_m). */
typedef struct fmoe_routing {
  const int32_t* topk_indx;
  const int32_t* gate_indx;
  const float* gate_scal;
  const int32_t* offs_raw;
  const int32_t* offs_pad; /* [E+1] tile offsets (prefill rasterization) */
  const int32_t* tile_map;
  const int32_t* n_tiles;
  int64_t n_tokens;
  int32_t top_k;
  int32_t n_experts;
  int32_t block_m;
  int32_t max_tiles;
} fmoe_routing;

/* GEMM1 with fused SiLU*mul: replaces matmul_ogs(x, w1, gather_indx, gammas)
 * + _silu_and_mul_triton (ops/fused_moe.py:189-202).  For every sorted slot
 * s of expert e:  inter = bf16(x[token(s)] @ w13[e]^T  [* gate_scal[s] when
 * gamma_on_input]);  act[s, j] = bf16(silu(inter[j]) * inter[N + j]).
 * act: [M*k, N] bf16 in sorted-slot order.  fp8 with prefill routing
 * (block_m >= 64): x is fp8 [M, K] with x_scale [M, K/128]; fp8 with decode
 * routing (block_m 16): x is bf16 and x_scale must be null (rows are
 * quantized in the kernel, bit-identical to fmoe_quant_fp8_group); int4:
 * w13_scale/w13_zero as in the header comment.
 * Requires K % 128 == 0, N % 128 == 0 (int4: group == 128). */
int fmoe_gemm1(int wtype, const void* x, const float* x_scale, const void* w13,
               const void* w13_scale, const void* w13_zero, int64_t K, int64_t N,
               const fmoe_routing* r, int gamma_on_input, void* act, int path, void* stream);

/* GEMM2: replaces matmul_ogs(act, w2, scatter_indx, gammas) up to the top-k
 * sum (ops/fused_moe.py:208-215): y[split][s, :] = act[s] @ w2[e]^T
 * [* gate_scal[s] when apply_gamma], fp32, sorted-slot order.  `splits`
 * partial sums over the reduction dim N are written to y[0..splits-1]
 * (fmoe_gemm2_splits() gives the count the library picks; every plane is
 * written, so y needs no clearing).  fp8 activations follow fmoe_gemm1:
 * fp8 act + act_scale with prefill routing, bf16 act + null act_scale with
 * decode routing. */
int fmoe_gemm2(int wtype, const void* act, const float* act_scale, const void* w2,
               const void* w2_scale, const void* w2_zero, int64_t K, int64_t N,
               const fmoe_routing* r, int apply_gamma, float* y, int splits, int path,
               void* stream);
int fmoe_gemm2_splits(int wtype, int64_t K, int64_t N, const fmoe_routing* r, int path);

/* Epilogue options of the bias / activation variants
 * (triton_kernel_fused_experts_with_bias, ops/fused_moe.py:219-309, and the
 * gelu branch of triton_kernel_fused_experts, :203-204).
 *   activation: enum fmoe_activation.
 *   bias: fp32 [E, rows] added to the fp32 GEMM result (GEMM1 rows = 2N in
 *     w13 row order, GEMM2 rows = K), or null.  With GEMM2 split-K the bias
 *     is added to split 0 only.
 *   alpha, limit (SWIGLU): with g = gate + b, l = linear + b, and when
 *     limit > 0: g = min(g, limit), l = clamp(l, -limit, limit);
 *     act = g * sigmoid(alpha * g) * (l + 1).  The routing weight (when
 *     applied on the input) multiplies the activation output.
 *   SILU / GELU round the GEMM1 result to bf16 before the activation (the
 *   reference runs them as a separate pass over a bf16 tensor); SWIGLU works
 *   on the fp32 result (the reference fuses it into matmul_ogs). */
typedef struct fmoe_epilogue {
  int32_t activation;
  const float* bias;
  float alpha;
  float limit;
} fmoe_epilogue;

/* fmoe_gemm1 / fmoe_gemm2 with an epilogue (null = SiLU, no bias). */
int fmoe_gemm1_ex(int wtype, const void* x, const float* x_scale, const void* w13,
                  const void* w13_scale, const void* w13_zero, int64_t K, int64_t N,
                  const fmoe_routing* r, int gamma_on_input, const fmoe_epilogue* ep, void* act,
                  int path, void* stream);
int fmoe_gemm2_ex(int wtype, const void* act, const float* act_scale, const void* w2,
                  const void* w2_scale, const void* w2_zero, int64_t K, int64_t N,
                  const fmoe_routing* r, int apply_gamma, const float* bias, float* y, int splits,
                  int path, void* stream);

/* Tile height the library pairs with the GEMM kernels for a problem size:
 * 16 selects the decode (streaming) kernels, 64 / 128 / 160 / 256 the prefill
 * kernels (256: bf16 only; 160 with fp8 weights needs K and N <= 8192 -- the
 * caller substitutes 128 above that; fmoe_fused_experts does so itself).
 * path: 0 = choose, 1 = prefill, 2 = decode (4-bit weights always report 16:
 * their large-batch route dequantizes to bf16 inside fmoe_fused_experts). */
int fmoe_choose_block_m(int wtype, int64_t M, int k, int E, int path);

/* The tile height fmoe_fused_experts uses for a layer of hidden size K and
 * intermediate size N: fmoe_choose_block_m with the fp8 160 -> 128 substitution
 * above applied (callers that build their own routing for the stage API use
 * this, so they always agree with the fused path).  Reference counterpart: the
 * block size triton_kernels' matmul_ogs picks for its routing, ops/fused_moe.py:190. */
int fmoe_fused_block_m(int wtype, int64_t M, int k, int E, int path, int64_t K, int64_t N);

/* Top-k combine (the scatter + sum inside matmul_ogs, ops/fused_moe.py:208-216,
 * and routed_scaling_factor, :399-404): out[t, :] = bf16(scale *
 * sum_{j<k} sum_{p<splits} y[p][gate_indx[t*k + j], :]), summed in fixed
 * order (deterministic). */
int fmoe_moe_sum(const float* y, int splits, const int32_t* gate_indx, int64_t M, int k,
                 int64_t K, float scale, void* out, void* stream);

/* ------------------------------------------------------ whole fused path
 * One call: align -> [fp8 quant x] -> GEMM1+SiLU -> [fp8 quant act] -> GEMM2
 * -> top-k sum.  Replaces triton_kernel_fused_experts + the routing
 * conversion (ops/fused_moe.py:103-216, :341-350, :399-404) with
 * SGLang-layout weights (no per-call transpose, cf. :326-327).  `path`:
 * 0 = choose, 1 = prefill (LDS-tiled) kernels, 2 = decode (streaming) kernels.
 * 4-bit weights (int4, MXFP4) run the decode kernels up to an average of 256
 * slots per expert; above it (or with path 1) the call first dequantizes both
 * weight tensors to bf16 inside the workspace (fmoe_fused_experts_workspace_bytes
 * then includes 2 * E * 3 * K * N bytes for them) and runs the bf16 prefill
 * kernels.
 */
typedef struct fmoe_fused_args {
  int32_t wtype;
  const void* x;
  int64_t M, K, N;
  int32_t E, top_k;
  const void* w13;
  const void* w2;
  const void* w13_scale;
  const void* w2_scale;
  const void* w13_zero;
  const void* w2_zero;
  int32_t group_size;
  const float* topk_weights;
  const int32_t* topk_ids;
  int32_t apply_router_weight_on_input;
  float routed_scaling_factor; /* 1.0 = none */
  int32_t path;
  void* out;
  void* workspace;
  size_t workspace_bytes;
  /* ABI version 2: epilogue of the bias / activation variants */
  int32_t activation;  /* enum fmoe_activation */
  const float* b13;    /* fp32 [E, 2N] or null */
  const float* b2;     /* fp32 [E, K] or null */
  float alpha;         /* SWIGLU */
  float limit;         /* SWIGLU clamp, <= 0 = none */
  const int32_t* expert_map; /* [n_global] global -> local expert (or -1), or null */
  int32_t n_global;          /* global expert count when expert_map is set */
} fmoe_fused_args;

size_t fmoe_fused_experts_workspace_bytes(const fmoe_fused_args* a);
int fmoe_fused_experts(const fmoe_fused_args* a, void* stream);

/* fmoe_fused_experts without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace is a library-owned device array of FMOE_NOALLOC_SCRATCH_BYTES
 * per GPU (held until the process ends; a->workspace / workspace_bytes are
 * ignored), looked up once per device with the calling thread's current
 * device, which must be the device of the tensors.  Calls whose workspace
 * query exceeds the maximum fail with FMOE_ERR_UNSUPPORTED (e.g. 4-bit
 * weights on the large-batch dequantize route: pass path = 2).  The kernels
 * need no zeroed scratch.  Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (different streams, threads) race. */
#define FMOE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int fmoe_fused_experts_noalloc(const fmoe_fused_args* a, void* stream);

/* ------------------------------------------------ checkpoint weight formats
 * Load-time repack of int4 MoE checkpoints into the FMOE_W_INT4 layout, once
 * per weight instead of per call (the reference re-lays weights out on every
 * forward, ops/fused_moe.py:326-327, and has no int4 path; the formats are
 * those SGLang loads for W4A16 MoE layers).  Per expert (stacked on a leading
 * E dim), K = reduction dim, N = output rows, g = group:
 *   FMOE_INT4_AWQ     qweight int32 [E, K, N/8], 8 columns per word in AutoAWQ
 *                     order (nibble i = column 8j + {0,2,4,6,1,3,5,7}[i]);
 *                     qzeros int32 [E, K/g, N/8] same packing; w = (q - z) * s
 *   FMOE_INT4_GPTQ_V1 qweight int32 [E, K/8, N] (nibble j of word i = row
 *                     8i + j); qzeros int32 [E, K/g, N/8] (nibble j = column
 *                     8c + j) holding zero - 1; no act-order (group of row k is
 *                     k / g)
 *   FMOE_INT4_GPTQ_V2 as V1 with the zero itself stored
 *   scales            fp16 [E, K/g, N] for all three
 * Outputs: q_out u8 [E, N, K/2], scales_out fp16 [E, K/g, N], zeros_out u8
 * [E, K/g, N/2] (the fmoe_gemm1 / fmoe_fused_experts int4 layout).
 * bad_zeros (device int32, optional, caller-zeroed) counts V1 zeros of 16,
 * which 4 bits cannot hold (they are stored as 0).  Needs N % 8 == 0,
 * g % 8 == 0 and K % g == 0. */
enum fmoe_int4_format {
  FMOE_INT4_AWQ = 0,
  FMOE_INT4_GPTQ_V1 = 1,
  FMOE_INT4_GPTQ_V2 = 2,
};
int fmoe_repack_int4(int format, const int32_t* qweight, const int32_t* qzeros,
                     const uint16_t* scales, int64_t E, int64_t K, int64_t N, int group,
                     uint8_t* q_out, uint16_t* scales_out, uint8_t* zeros_out,
                     int32_t* bad_zeros, void* stream);

/* Load-time tiling of FMOE_W_INT4 weights into FMOE_W_INT4_TILED (and of
 * FMOE_W_MXFP4 weight bytes, packed the same way, into FMOE_W_MXFP4_TILED).  No
 * counterpart in the reference (its W4A16 kernels read the row-major
 * layout on every call); for callers that prepare weights once, as after
 * fmoe_repack_int4.  q [E, R, K/2] u8 (row r, element 2i low nibble) ->
 * out [E, R/16, K/128, 1024]: block (b, c) holds rows 16b..16b+15, bytes
 * 64c..64c+63 of each (one 128-element quant group), byte 16 (16 g + r) + i
 * = byte 64c + 16g + i of row 16b + r.  A decode wave's 16-row x 64-byte
 * weight load is then one contiguous 1 KiB read.  Needs R % 16 == 0 and
 * K % 128 == 0; q and out must not overlap. */
int fmoe_tile_int4(const uint8_t* q, int64_t E, int64_t R, int64_t K, uint8_t* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FMOE_H_ */
