/*
 * dsmoe — MI355X (gfx950) MoE-FFN layer of jbreams/deepseek-rs as a C ABI.
 *
 * The reference's "MoE-layer API" is the launch surface of its kernel
 * modules as called by Session::decode_attn_out_and_ffn
 * (engine/src/session.rs:1894-2155).  This header replaces that surface:
 * one whole-layer call (dsmoe_forward) plus one entry point per reference
 * kernel, each citing the launcher it replaces.
 *
 * Conventions
 *   - Every pointer argument is a DEVICE pointer unless its name ends in
 *     _host.  Weights are the raw GGUF block bytes, in the GGUF layout:
 *       router   f16   [E][d]
 *       gate/up  IQ2_XXS [E][I][d/256] x 66 B
 *       down     Q2_K  [E][d][I/256] x 84 B
 *       shared   Q8_0  [I_s][d/32] x 34 B (gate, up), [d][I_s/32] (down)
 *                or IQ2_XXS/Q2_K like the routed experts (shared_fmt = 1)
 *     Weight and activation base pointers must be 16-byte aligned.
 *   - All calls are asynchronous on `stream` (a hipStream_t; NULL = the
 *     default stream) and do no host synchronisation, like the reference's
 *     launches on its single CudaStream.
 *   - Return 0 on success; otherwise a DSMOE_ERR_* code, with a message
 *     from dsmoe_last_error() (per host thread).  Shape errors are detected
 *     before anything is launched.
 *   - A dsmoe_ctx owns its scratch buffers and is not thread-safe: use one
 *     per stream, as the reference uses one Session per stream.
 */
#ifndef DSMOE_H
#define DSMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* dsmoe_stream_t; /* hipStream_t */
typedef struct dsmoe_ctx dsmoe_ctx;

enum {
  DSMOE_OK = 0,
  DSMOE_ERR_INVALID = 1,     /* bad argument / shape / null pointer */
  DSMOE_ERR_UNSUPPORTED = 2, /* valid but outside what the kernels handle */
  DSMOE_ERR_HIP = 3,         /* HIP runtime error */
  DSMOE_ERR_NOMEM = 4,       /* device allocation failed */
  DSMOE_ERR_MODULE = 5,      /* kernel code object missing / unloadable */
  DSMOE_ERR_NOT_FOUND = 6    /* GGUF tensor or key absent */
};

/* Layer configuration.  The reference hard-codes d=4096, I=2048, E=256,
 * k=6, route_scale=1.5, clamp=10 (engine/src/model.rs:15-26,
 * session.rs:21); here they are runtime parameters.  n_group = 1 is the
 * reference's routing; n_group > 1 adds group-limited top-k. */
typedef struct dsmoe_config {
  int32_t d_model;     /* multiple of 512, at most 8192 */
  int32_t d_ff;        /* routed expert intermediate, multiple of 256 */
  int32_t n_expert;    /* 1..1024 (the batch path needs <= 512; above, every T runs the matvec launches) */
  int32_t top_k;       /* 1..32 */
  int32_t n_group;     /* 1 = reference routing; else divides n_expert, <= 64 */
  int32_t topk_group;  /* groups kept when n_group > 1 */
  float route_scale;   /* weights sum to this (1.5 in the reference) */
  float swiglu_clamp;  /* SWIGLU_CLAMP = 10 in the reference; <= 1e-6 disables */
  int32_t has_bias;    /* correction bias added for selection only */
  int32_t shared_fmt;  /* 0 = Q8_0 (reference), 1 = IQ2_XXS/Q2_K, -1 = none */
  int32_t d_ff_shared; /* shared expert intermediate (multiple of 64; of 256 if shared_fmt = 1) */
} dsmoe_config;

typedef struct dsmoe_weights {
  const void* router_f16; /* blk.N.ffn_gate_inp   */
  const float* bias;      /* blk.N.exp_probs_b (f32 [E]) or NULL */
  const void* gate;       /* blk.N.ffn_gate_exps  */
  const void* up;         /* blk.N.ffn_up_exps    */
  const void* down;       /* blk.N.ffn_down_exps  */
  const void* sh_gate;    /* blk.N.ffn_gate_shexp */
  const void* sh_up;      /* blk.N.ffn_up_shexp   */
  const void* sh_down;    /* blk.N.ffn_down_shexp */
  /* Optional, no reference counterpart: the Q8_0 shared expert's gate, up
   * and down already rewritten by dsmoe_q8_0_unpack (codes f16 [rows *
   * in_dim], scales f32 [rows * in_dim / 32]), done once per weight load.
   * Batches on the wide shared-expert path (T >= 1024) then read these
   * instead of unpacking the three matrices on every call.  All six NULL
   * (a zero-initialised struct) = unpack per call. */
  const uint16_t* sh_codes[3];
  const float* sh_scales[3];
} dsmoe_weights;

const char* dsmoe_version(void);
const char* dsmoe_last_error(void);

/* Loads the kernel code object on the current device (idempotent).  NULL
 * = dsmoe_kernels.hsaco next to this library.  Called implicitly by every
 * entry point; exposed so a caller can fail early, as Kernels::load does
 * (engine/src/engine.rs:31-55). */
int dsmoe_init(const char* code_object_path);

/* --------------------------------------------------------------------- */
/* Whole layer                                                            */
/* --------------------------------------------------------------------- */
/* Scratch for up to max_tokens tokens (Session::new, session.rs:260-271). */
int dsmoe_create(const dsmoe_config* cfg, int32_t max_tokens, dsmoe_ctx** out);
int dsmoe_destroy(dsmoe_ctx* ctx);
/* Bytes of device scratch the context holds. */
size_t dsmoe_scratch_bytes(const dsmoe_ctx* ctx);

/* The MoE FFN of one layer for T tokens (session.rs:1894-2155):
 *   x          f32 [T][d]   (ffn_norm)
 *   shared_out f32 [T][d]   shared expert output
 *   routed_out f32 [T][d]   sum over the k routed experts in slot order
 *   selected   i32 [T][k], weights f32 [T][k]: routing, optional (NULL)
 * hc_expand's input is shared_out + routed_out (session.rs:2157-2175).
 * T <= 8 runs three launches (router logits + quantized x | routing, routed
 * and shared gate/up and quantized mid | routed and shared down); larger T
 * sorts the pairs by expert and runs grouped GEMMs.  T = 0 returns
 * DSMOE_OK without reading or writing anything (the token buffers may then be
 * NULL).  Calls that overlap on one context race (they share its scratch and
 * row counters). */
int dsmoe_forward(dsmoe_ctx* ctx, const dsmoe_weights* w, const float* x, int32_t T,
                  float* shared_out, float* routed_out, int32_t* selected, float* weights,
                  dsmoe_stream_t stream);

/* dsmoe_forward for T <= 8 without a context and without allocating: no
 * counterpart in the reference.  For callers that cannot allocate device
 * memory (code under graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The scratch between the launches is a static 16 MiB
 * device array per GPU, set up when the library loads its kernels on that
 * device (dsmoe_init or the first call); a layer whose scratch for 8 tokens
 * exceeds it (or T > 8) is rejected with DSMOE_ERR_UNSUPPORTED.  Same
 * arguments and results as dsmoe_forward.  All calls on one GPU share the
 * array: calls that overlap on one GPU (two streams, two threads) race.
 * Graph capture: the per-device set-up launches a clear and synchronizes,
 * so it must run before capture (dsmoe_init, or one eager call on that
 * device); a first call on a capturing stream returns DSMOE_ERR_INVALID. */
int dsmoe_forward_noalloc(const dsmoe_config* cfg, const dsmoe_weights* w, const float* x, int32_t T,
                          float* shared_out, float* routed_out, int32_t* selected, float* weights,
                          dsmoe_stream_t stream);

/* Hash routing for the layers that route by token id (the reference's
 * hash_mode, moe.rs:92-109, with the table blk.N.ffn_gate_tid2eid): when
 * `hash` (device, i32 [hash_rows][top_k]) is set, every later dsmoe_forward
 * on this context takes the experts of token t from row tokens[t] of the
 * table (tokens: device i32 [T], read at each forward; NULL = row 0) instead
 * of the top-k selection; the weights are computed as in
 * dsmoe_router_select_hash.  hash = NULL returns to top-k routing. */
int dsmoe_set_hash_routing(dsmoe_ctx* ctx, const int32_t* hash, int32_t hash_rows, const int32_t* tokens);

/* Per-stage timing of dsmoe_forward (no reference counterpart: the
 * reference has no tracing).  When enabled, every stage of the forward is
 * bracketed by hipEvents on the caller's stream; dsmoe_profile_read waits
 * for them and returns the accumulated milliseconds and launch counts per
 * stage (arrays of DSMOE_STAGE_COUNT), optionally resetting them.
 * Without profiling, batches on the wide shared-expert path run the shared
 * expert's GEMMs on a second stream of the context, concurrent with the
 * routed experts; with profiling on, all stages run on the caller's stream,
 * one after another, so each stage's time is its own. */
enum {
  DSMOE_STAGE_PREP = 0,   /* router logits + Q8_K(x) + Q8_0(x)            */
  DSMOE_STAGE_SELECT,     /* routing                                      */
  DSMOE_STAGE_UP,         /* routed + shared gate/up/SwiGLU               */
  DSMOE_STAGE_MIDQ,       /* activation quantization of the SwiGLU output */
  DSMOE_STAGE_DN,         /* routed down + slot sum + shared down         */
  /* inside UP / DN on the grouped path (T > 8) */
  DSMOE_STAGE_GU_GROUPED, /* routed gate/up/SwiGLU grouped GEMM            */
  DSMOE_STAGE_SH_UP,      /* shared gate/up/SwiGLU GEMM                    */
  DSMOE_STAGE_DN_GROUPED, /* routed down grouped GEMM (before the slot sum) */
  DSMOE_STAGE_SH_DN,      /* shared down GEMM                              */
  DSMOE_STAGE_COUNT
};
const char* dsmoe_stage_name(int32_t stage);
int dsmoe_set_profiling(dsmoe_ctx* ctx, int32_t enable);
int dsmoe_profile_read(dsmoe_ctx* ctx, double* total_ms, int64_t* launches, int32_t reset);

/* --------------------------------------------------------------------- */
/* Per-kernel entry points (the reference launch surface)                 */
/* --------------------------------------------------------------------- */
/* matmul_f16 (engine/src/kernels/matmul.rs:57-105): out[t][e] = sum_i
 * f16(w[e][i]) x[t][i], 256 strided partials + halving tree; d a multiple
 * of 256, at most 65536. */
int dsmoe_router_logits(const uint16_t* w, const float* x, float* out, int32_t d, int32_t E, int32_t T,
                        dsmoe_stream_t stream);

/* router_select_parallel (engine/src/kernels/moe.rs:177-287): probs =
 * sqrt(softplus(logits)); top-k by (probs + bias); weights = probs of the
 * selection / (max(sum, 2^-14) / route_scale).  probs may be NULL. */
int dsmoe_router_select(const dsmoe_config* cfg, const float* logits, const float* bias, int32_t T,
                        float* probs, int32_t* selected, float* weights, dsmoe_stream_t stream);

/* q8k_quantize (engine/src/kernels/quantize.rs:309-417): rows x in_dim f32
 * -> rows x in_dim/256 Q8_K blocks of 292 B. */
int dsmoe_q8k_quantize(const float* x, void* out, int32_t in_dim, int32_t rows, dsmoe_stream_t stream);

/* q8k_quantize as above, also writing the quantized values as f16
 * [rows][in_dim] (out_h): the activation operand of the grouped MFMA
 * kernels.  The f16 copy has no reference counterpart. */
int dsmoe_q8k_quantize_h(const float* x, void* out, uint16_t* out_h, int32_t in_dim, int32_t rows,
                         dsmoe_stream_t stream);

/* q8k_quantize as above, also writing the quantized values as int8
 * [rows][in_dim] (out_i8, 16-byte aligned) and the sum of each 16-element
 * group as f16 [rows][in_dim/16] (bsum_h; the bsums of the Q8_K block, exact
 * in f16): the activation operands of the int8 grouped down.  The two
 * copies have no reference counterpart. */
int dsmoe_q8k_quantize_i8(const float* x, void* out, int8_t* out_i8, uint16_t* bsum_h, int32_t in_dim, int32_t rows,
                          dsmoe_stream_t stream);

/* quantize_q8_0 as below, also writing the codes as f16 [rows][in_dim]
 * (out_h; no reference counterpart): the operand of dsmoe_q8_0_gemm. */
int dsmoe_q8_0_quantize_h(const float* x, int8_t* xq, float* xscale, uint16_t* out_h, int32_t in_dim, int32_t rows,
                          dsmoe_stream_t stream);

/* quantize_q8_0 (engine/src/kernels/quantize.rs:147-225). */
int dsmoe_q8_0_quantize(const float* x, int8_t* xq, float* xscale, int32_t in_dim, int32_t rows,
                        dsmoe_stream_t stream);

/* moe_gate_up_mid_qwarp32 (engine/src/kernels/moe.rs:622-715): for pair =
 * t*k + slot and row < I, gate/up = IQ2_XXS row . Q8_K x[t], clamped;
 * mid = silu(gate) * up * weights[pair].  gate_out/up_out may be NULL.
 * E = experts in gate/up: an id outside [0, E) reads expert 0 (the
 * reference's -1 for an unfilled slot does the same; it checks no upper
 * bound).  selected NULL = expert 0 for every pair, weights NULL = 1. */
int dsmoe_gate_up_mid(const void* gate, const void* up, const void* xq, const int32_t* selected,
                      const float* weights, float* gate_out, float* up_out, float* mid_out, int32_t d,
                      int32_t I, int32_t T, int32_t k, int32_t E, float clamp, dsmoe_stream_t stream);

/* moe_gate_up_mid_sorted_qwarp32 (engine/src/kernels/moe.rs:721-815):
 * the pairs grouped by expert by dsmoe_dispatch with block_m =
 * DSMOE_GROUPED_TILE_M; mid_out[pair][row] as dsmoe_gate_up_mid computes it
 * up to f32 rounding of the order in which a row's superblock values are
 * added (superblocks in order here, per-lane partials and a butterfly in the
 * reference; each superblock's integer sum and block value are the
 * reference's).  xh/xq: Q8_K(x) from dsmoe_q8k_quantize_h.  weights: routing
 * weight per pair (NULL = 1).  Runs on the matrix cores (f16 operands holding
 * the exact integer codes, f32 accumulation); I a multiple of 256. */
#define DSMOE_GROUPED_TILE_M 64
int dsmoe_gate_up_mid_sorted(const void* gate, const void* up, const uint16_t* xh, const void* xq,
                             const uint32_t* sorted_pairs, const uint32_t* offsets, const uint32_t* tile_offsets,
                             const uint32_t* tile_experts, const uint32_t* tile_starts, const float* weights,
                             float* mid_out, int32_t d, int32_t I, int32_t k, int32_t E, int32_t pairs, float clamp,
                             dsmoe_stream_t stream);

/* moe_gate_up_mid_sorted_qwarp32 (engine/src/kernels/moe.rs:721-815) in
 * the expert-major matvec form, for batches with few pairs per expert: the
 * pairs grouped by dsmoe_dispatch with block_m (1..DSMOE_EM_TILE_M); every
 * expert's weight rows stream once per tile of up to block_m pairs, each
 * decoded block multiplied with all the tile's activations.  xq: Q8_K(x).
 * Same bits as dsmoe_gate_up_mid.  d a multiple of 512 whose block_m
 * activations fit the workgroup's LDS (block_m 8: d <= 7168). */
#define DSMOE_EM_TILE_M 8
int dsmoe_gate_up_mid_em(const void* gate, const void* up, const void* xq, const uint32_t* sorted_pairs,
                         const uint32_t* offsets, const uint32_t* tile_offsets, const uint32_t* tile_experts,
                         const uint32_t* tile_starts, const float* weights, float* mid_out, int32_t d, int32_t I,
                         int32_t k, int32_t E, int32_t pairs, int32_t block_m, float clamp, dsmoe_stream_t stream);

/* moe_down_sorted_qwarp32 (moe.rs:871-916) in the expert-major form:
 * down_out[pair][row] for the pairs grouped by dsmoe_dispatch with block_m
 * (1..DSMOE_EM_TILE_M); mq: Q8_K(mid).  Same bits as dsmoe_down's per-pair
 * values; the slot sum is dsmoe_moe_sum.  I at most 2048. */
int dsmoe_down_em(const void* down, const void* mq, const uint32_t* sorted_pairs, const uint32_t* offsets,
                  const uint32_t* tile_offsets, const uint32_t* tile_experts, const uint32_t* tile_starts,
                  float* down_out, int32_t d, int32_t I, int32_t E, int32_t pairs, int32_t block_m,
                  dsmoe_stream_t stream);

/* moe_down_sorted_qwarp32 (engine/src/kernels/moe.rs:821-916, sorted
 * variant): down_out[pair][row] for the pairs grouped by dsmoe_dispatch
 * (block_m = DSMOE_GROUPED_TILE_M), the per-pair values dsmoe_down computes
 * up to f32 rounding of the order in which a row's superblock values are
 * added (each superblock's integer sums and block value are the
 * reference's); m8/bsum_h/mq: Q8_K(mid) from dsmoe_q8k_quantize_i8.  The
 * slot sum is dsmoe_moe_sum.  int8 matrix cores (weights sc * q and the mid
 * codes are exact int8, each superblock's isum an exact int32); d a multiple
 * of 256. */
int dsmoe_down_sorted(const void* down, const int8_t* m8, const uint16_t* bsum_h, const void* mq,
                      const uint32_t* sorted_pairs, const uint32_t* offsets, const uint32_t* tile_offsets,
                      const uint32_t* tile_experts, const uint32_t* tile_starts, float* down_out, int32_t d, int32_t I,
                      int32_t E, int32_t pairs, dsmoe_stream_t stream);

/* moe_down_qwarp32 + moe_sum / moe_down_sum6_qwarp32 (engine/src/kernels/
 * moe.rs:821-866, :922-1005): down_out[pair][row] = Q2_K row . Q8_K
 * midq[pair]; out[t][row] = slot-ordered sum.  Either output may be NULL.
 * E and ids outside [0, E) as for dsmoe_gate_up_mid. */
int dsmoe_down(const void* down, const void* midq, const int32_t* selected, float* down_out, float* out,
               int32_t d, int32_t I, int32_t T, int32_t k, int32_t E, dsmoe_stream_t stream);

/* moe_sum (engine/src/kernels/moe.rs:983-1005). */
int dsmoe_moe_sum(const float* down, float* out, int32_t d, int32_t k, int32_t T, dsmoe_stream_t stream);

/* Peak probes, no reference counterpart (measurement support for the
 * benchmark).  kind 0: dense f16 MFMA, 2 workgroups of 4 waves per CU, each
 * wave `iters` rounds of 8 independent v_mfma_f32_32x32x16_f16 (32768 flops
 * each).  kind 1: one read of `bytes` of `src` (device, 16-byte aligned)
 * with 16-byte loads, 8 workgroups per CU.  `sink` (device, >= 8 floats per
 * CU) is written only on a data-dependent branch. */
int dsmoe_probe(int32_t kind, const void* src, size_t bytes, int64_t iters, float* sink, dsmoe_stream_t stream);

/* router_select with hash_mode = 1 (engine/src/kernels/moe.rs:92-109,
 * weights :143-159): selected[t][j] = hash[tok][j] with tok = tokens[t]
 * (token_scalar when tokens is NULL; an id outside [0, hash_rows) uses row
 * 0); probs as in dsmoe_router_select; weight j = probs[t][selected] (0 for
 * an id outside [0, n_expert)) / (max(sum in slot order, 2^-14) /
 * route_scale).  The reference hard-codes k = 6, E = 256, scale 1.5; here
 * they come from cfg.  The correction bias plays no part. */
int dsmoe_router_select_hash(const dsmoe_config* cfg, const float* logits, const int32_t* hash, int32_t hash_rows,
                             const int32_t* tokens, int32_t token_scalar, int32_t T, float* probs,
                             int32_t* selected, float* weights, dsmoe_stream_t stream);

/* The HC FFN pre-norm that produces the layer's input (session.rs:1830-1892):
 * rms_norm_plain of the HC residual streams (engine/src/kernels/norm.rs:14-63),
 * hc_mix = dsmoe_router_logits of it with the [24][n_hc * n_embd] f16
 * hc_ffn_fn matrix (matmul_f16), then dsmoe_hc_split_norm. */
/* rms_norm_plain: out[r][i] = x[r][i] * 1 / sqrt(sum of squares / n + eps),
 * the sum over 256 lane-strided partials and a halving tree. */
int dsmoe_rms_norm_plain(const float* x, float* out, int32_t n, int32_t rows, float eps, dsmoe_stream_t stream);
/* hc_split_weighted_sum_norm_fused (engine/src/kernels/hc.rs:313-398, with
 * hc4_split_one :17-99), n_hc = 4: per row the 24-value split (pre =
 * sigmoid + eps, post = 2 sigmoid, comb = row softmax + eps, column
 * normalisation and sinkhorn_iters - 1 Sinkhorn rounds) into split[row],
 * out = sum_h residual_hc[row][h] * pre[h] (ffn_cur) and norm_out = out *
 * 1 / sqrt(mean square + norm_eps) * norm_w (ffn_norm, the input of
 * dsmoe_forward).  The exponentials are this library's expf. */
int dsmoe_hc_split_norm(const float* mix, const float* scale, const float* base, const float* residual_hc,
                        const float* norm_w, float* split, float* out, float* norm_out, int32_t n_embd, int32_t n_hc,
                        int32_t n_rows, int32_t sinkhorn_iters, float eps, float norm_eps, dsmoe_stream_t stream);

/* hc_expand (engine/src/kernels/hc.rs:212-259), the FFN residual merge that
 * consumes the layer's outputs (session.rs:2157-2175: block_out =
 * shared_out, block_add = routed_out, has_add = 1 after a MoE layer):
 *   out_hc[t][dst][i] = (block_out[t][i] (+ block_add[t][i])) * post[dst]
 *                       + sum_src comb[dst + src*n_hc] * residual_hc[t][src][i]
 * with post = split[t*mix_hc + n_hc ..] and comb = split[t*mix_hc + 2*n_hc ..].
 * block_add may be NULL when has_add = 0. */
int dsmoe_hc_expand(const float* block_out, const float* block_add, const float* residual_hc, const float* split,
                    float* out_hc, int32_t n_embd, int32_t n_hc, int32_t n_tokens, int32_t mix_hc, int32_t has_add,
                    dsmoe_stream_t stream);

/* matmul_q8_0_preq_warp8 / _batch_warp8 (engine/src/kernels/matmul.rs:357-458).
 * in_dim a multiple of 64. */
int dsmoe_q8_0_matvec(const void* w, const int8_t* xq, const float* xscale, float* out, int32_t in_dim,
                      int32_t out_dim, int32_t T, dsmoe_stream_t stream);

/* matmul_q8_0_preq_batch_warp8 (engine/src/kernels/matmul.rs:412-458) as a
 * GEMM for the whole batch: out[t][row] = Q8_0 row . Q8_0(x[t]) with the
 * reference's per-row arithmetic (same bits as dsmoe_q8_0_matvec).  With
 * w1 (the up matrix) the output is swiglu(w0 . x, w1 . x) with weight 1 and
 * the clamp (utils.rs:141-163), as the shared expert's gate/up.  xh/xscale
 * from dsmoe_q8_0_quantize_h.  out_dim a multiple of 32 (two matrices) or
 * 64.  Matrix cores, exact integer codes in f16. */
int dsmoe_q8_0_gemm(const void* w0, const void* w1, const uint16_t* xh, const float* xscale, float* out, int32_t in_dim,
                    int32_t out_dim, int32_t T, float clamp, dsmoe_stream_t stream);

/* The shared-expert GEMM for large batches, no reference counterpart in
 * form (the products of matmul_q8_0_preq_batch_warp8, matmul.rs:412-458).
 * dsmoe_q8_0_unpack rewrites a Q8_0 matrix [rows][in_dim/32 blocks] into
 * the operand layout of dsmoe_q8_0_gemm_unpacked: codes as f16
 * (rows * in_dim of them) and block scales as f32 (rows * in_dim / 32); an
 * engine can do this once per weight load.  rows a multiple of 16, in_dim of
 * 64; codes 16-byte and w 4-byte aligned.
 * dsmoe_q8_0_gemm_unpacked is dsmoe_q8_0_gemm over unpacked matrices (w1h /
 * w1s NULL for one matrix) with each block's value (d_w * d_x) * sum added
 * to the running sum in block order by one fma, where the reference adds
 * 32 lane-strided partials and then halves them: equal to dsmoe_q8_0_gemm up
 * to f32 rounding of that order (the integer sums are the same).  in_dim a
 * multiple of 64, at most 8192; out_dim a multiple of 128 (one matrix) or 64
 * (two); xh and out 16-byte aligned.  Full speed from about 1024 tokens (a
 * workgroup takes 256 tokens). */
int dsmoe_q8_0_unpack(const void* w, int32_t rows, int32_t in_dim, uint16_t* codes, float* scales,
                      dsmoe_stream_t stream);
int dsmoe_q8_0_gemm_unpacked(const uint16_t* w0h, const float* w0s, const uint16_t* w1h, const float* w1s,
                             const uint16_t* xh, const float* xscale, float* out, int32_t in_dim, int32_t out_dim,
                             int32_t T, float clamp, dsmoe_stream_t stream);

/* swiglu (engine/src/kernels/utils.rs:141-163). */
int dsmoe_swiglu(const float* gate, const float* up, float* out, int32_t n, float clamp, float weight,
                 dsmoe_stream_t stream);

/* moe_count_sorted_pairs + moe_prefix_sorted_pairs + moe_scatter_sorted_pairs
 * + moe_build_expert_tile_offsets/tiles (engine/src/kernels/moe.rs:299-362,
 * :547-596).  The scatter is stable (ascending pair order within an expert).
 * tile_* may be NULL; tile_experts/starts need room for
 * pairs/block_m + E entries.  E <= 512. */
int dsmoe_dispatch(const int32_t* selected, int32_t pairs, int32_t E, int32_t block_m, uint32_t* counts,
                   uint32_t* offsets, uint32_t* sorted_pairs, uint32_t* tile_offsets,
                   uint32_t* tile_experts, uint32_t* tile_starts, dsmoe_stream_t stream);

/* --------------------------------------------------------------------- */
/* Synthetic tensors (no reference counterpart: the reference loads       */
/* pre-quantized GGUF weights).  N(0, sigma) values from (seed, tensor_id,  */
/* element) quantized to fmt; zero outside rows_real x cols_real.  The     */
/* device and host variants produce identical bytes.                      */
/* --------------------------------------------------------------------- */
enum { DSMOE_FMT_IQ2_XXS = 0, DSMOE_FMT_Q2_K = 1, DSMOE_FMT_Q8_0 = 2, DSMOE_FMT_F16 = 3, DSMOE_FMT_F32 = 4 };
size_t dsmoe_tensor_bytes(int32_t fmt, int64_t n_mats, int32_t rows, int32_t cols);
int dsmoe_synth_tensor(void* out, int32_t fmt, uint64_t seed, uint64_t tensor_id, int64_t n_mats, int32_t rows,
                       int32_t cols, int32_t rows_real, int32_t cols_real, float sigma, dsmoe_stream_t stream);
int dsmoe_synth_tensor_host(void* out_host, int32_t fmt, uint64_t seed, uint64_t tensor_id, int64_t n_mats,
                            int32_t rows, int32_t cols, int32_t rows_real, int32_t cols_real, float sigma,
                            int32_t nthreads);

/* --------------------------------------------------------------------- */
/* GGUF expert tensors (engine/src/gguf.rs, engine/src/model.rs:28-104)    */
/* --------------------------------------------------------------------- */
/* A read-only GGUF v2/v3 file, memory-mapped: the metadata section is
 * walked (values skipped by type; an unknown metadata type, tensor type, bad
 * magic, a version outside 2..3, or a tensor past the end of the file is
 * DSMOE_ERR_INVALID), tensor infos are read, and the data section starts at
 * the next 32-byte boundary after them.  Tensor data are host pointers into
 * the mapping, valid until dsmoe_gguf_close; the caller copies what it needs
 * to the device. */
typedef struct dsmoe_gguf dsmoe_gguf;
enum { DSMOE_GGUF_F32 = 0, DSMOE_GGUF_F16 = 1, DSMOE_GGUF_Q8_0 = 8, DSMOE_GGUF_Q2_K = 10, DSMOE_GGUF_Q4_K = 12,
       DSMOE_GGUF_IQ2_XXS = 16, DSMOE_GGUF_I32 = 26 };
typedef struct dsmoe_gguf_tensor {
  const char* name;  /* owned by the file handle */
  int32_t type;      /* DSMOE_GGUF_* */
  int32_t n_dims;    /* 1..4; unused dims read 1 */
  uint64_t dims[4];  /* as stored in the file */
  uint64_t offset;   /* from the start of the data section */
  uint64_t bytes;    /* TensorType::byte_size of the element count (model.rs:80-85) */
  const void* data;  /* host pointer into the mapping */
} dsmoe_gguf_tensor;
int dsmoe_gguf_open(const char* path, dsmoe_gguf** out);
int dsmoe_gguf_close(dsmoe_gguf* g);
int64_t dsmoe_gguf_tensor_count(const dsmoe_gguf* g);
uint64_t dsmoe_gguf_data_offset(const dsmoe_gguf* g);
int dsmoe_gguf_tensor_at(const dsmoe_gguf* g, int64_t index, dsmoe_gguf_tensor* out);
/* GgufFile::find; DSMOE_ERR_NOT_FOUND when no tensor has the name. */
int dsmoe_gguf_find(const dsmoe_gguf* g, const char* name, dsmoe_gguf_tensor* out);
/* GgufFile::read_kv_u32 / read_kv_i32_array (a key of another type is not
 * found; *count is the array length, at most cap values are copied). */
int dsmoe_gguf_kv_u32(const dsmoe_gguf* g, const char* key, uint32_t* out);
int dsmoe_gguf_kv_i32_array(const dsmoe_gguf* g, const char* key, int32_t* out, int64_t cap, int64_t* count);
/* The MoE tensors of one layer, by the engine's names (engine.rs:175-187):
 * out[0..9] = blk.N.{ffn_gate_inp.weight, exp_probs_b.bias,
 * ffn_gate_exps.weight, ffn_up_exps.weight, ffn_down_exps.weight,
 * ffn_gate_shexp.weight, ffn_up_shexp.weight, ffn_down_shexp.weight,
 * ffn_gate_tid2eid.weight, ffn_norm.weight}; bit i of *present says out[i]
 * was found (absent entries are zeroed). */
#define DSMOE_GGUF_MOE_TENSORS 10
int dsmoe_gguf_moe_layer(const dsmoe_gguf* g, int32_t layer, dsmoe_gguf_tensor* out, int32_t* present);

#ifdef __cplusplus
}
#endif
#endif
