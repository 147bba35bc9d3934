// Kernel argument blocks.  Every kernel in dsmoe_kernels.hip takes exactly
// one of these structs by value; the host launcher (dsmoe_host.cpp) fills it
// and passes it through hipModuleLaunchKernel.  Plain C layout, identical on
// both sides of the boundary.
#pragma once
#include <stdint.h>

namespace dsm {

struct RouterLogitsArgs {
  const uint16_t* w;  // [E][d] f16 bits
  const float* x;     // [T][d]
  float* out;         // [T][E]
  int32_t d, E, T;
};

struct RouterSelectArgs {
  const float* logits;  // [T][E]
  const float* bias;    // [E] or null
  float* probs;         // [T][E] or null
  int32_t* selected;    // [T][k]
  float* weights;       // [T][k]
  int32_t T, E, k, n_group, topk_group, has_bias;
  float route_scale;
};

// Hash routing (moe.rs:92-109): experts from a token-id table.
struct HashSelectArgs {
  const float* logits;    // [T][E]
  const int32_t* hash;    // [hash_rows][k]
  const int32_t* tokens;  // [T] or null (token_scalar for every token)
  float* probs;           // [T][E] or null
  int32_t* selected;      // [T][k]
  float* weights;         // [T][k]
  int32_t token_scalar, hash_rows, T, E, k;
  float route_scale;
};

struct Q8KArgs {
  const float* x;  // [rows][in_dim]
  uint8_t* out;    // [rows][in_dim/256] x 292 B
  int32_t in_dim, rows;
  uint16_t* out_h = nullptr;  // optional: the qs again as f16 [rows][in_dim] (MFMA operand)
  int8_t* out_8 = nullptr;    // optional: the qs again as int8 [rows][in_dim] (int8 MFMA operand)
  uint16_t* bsum_h = nullptr; // optional: the 16-element sums as f16 [rows][in_dim/16]
};

struct Q80Args {
  const float* x;   // [rows][in_dim]
  int8_t* xq;       // [rows][nb*32]
  float* xscale;    // [rows][nb]
  int32_t in_dim, rows;
  uint16_t* out_h = nullptr;  // optional: the codes again as f16 [rows][nb*32] (MFMA operand)
};

// The wave-per-block quantization forms read x as 16-byte vectors and store
// the codes as 4-byte words and their f16 copies as 8-byte words; other
// alignments (and Q8_0 rows that are not a multiple of 32) take the
// workgroup-per-block forms.
inline __host__ __device__ bool q8k_waves_ok(const Q8KArgs& q) {
  return ((uintptr_t)q.x & 15) == 0 && ((uintptr_t)q.out & 3) == 0 && ((uintptr_t)q.out_h & 7) == 0;
}
inline __host__ __device__ bool q80_waves_ok(const Q80Args& q) {
  return q.in_dim % 32 == 0 && ((uintptr_t)q.x & 15) == 0 && ((uintptr_t)q.xq & 3) == 0 &&
         ((uintptr_t)q.out_h & 7) == 0;
}

// Routed gate/up/SwiGLU over IQ2_XXS.  Work list entry = pair index
// (pair = tok*k + slot); when `pair_list` is null, blockIdx.y is the pair.
struct GateUpArgs {
  const uint8_t* gate;     // [E][I][d/256] x 66 B
  const uint8_t* up;
  const uint8_t* xq;       // Q8_K [T][d/256]
  const int32_t* selected; // [T*k] (null: expert 0, weight 1: shared expert); ids outside [0,E) read expert 0
  const float* weights;    // [T*k] (null: weight 1)
  const uint32_t* pair_list;
  float* gate_out;         // [pairs][I] or null
  float* up_out;           // [pairs][I] or null
  float* mid_out;          // [pairs][I]
  int32_t d, I, k, rows_per_wg, E;
  float clamp;
};

// Down projection over Q2_K, summed over the k slots of one token in slot
// order; blockIdx.y = token.  When `down_out` is set the per-pair values are
// written too ([pairs][d]).
struct DownArgs {
  const uint8_t* down;      // [E][d][I/256] x 84 B
  const uint8_t* midq;      // Q8_K [T*k][I/256]
  const int32_t* selected;  // [T*k] (null: expert 0); ids outside [0,E) read expert 0
  float* out;               // [T][d] or null
  float* down_out;          // [T*k][d] or null
  int32_t d, I, k, rows_per_wg, E;
};

// Q8_0 x Q8_0-activation matvec (shared expert), optionally two matrices
// (gate and up) fused with SwiGLU.
struct Q80MatvecArgs {
  const uint8_t* w0;      // [out][nb] x 34 B
  const uint8_t* w1;      // second matrix (up) or null
  const int8_t* xq;       // [T][nb*32]
  const float* xscale;    // [T][nb]
  float* out0;            // [T][out] (gate, or the single product)
  float* out1;            // [T][out] (up) or null
  float* mid;             // [T][out] swiglu(out0, out1) or null
  int32_t in_dim, out_dim, rows_per_wg;
  float clamp;
};

// Fused launches: one grid whose workgroups take different roles, by
// contiguous blockIdx.x ranges ("n_*" = workgroups of each role, a zero
// count disables the role).  Every role reads threadIdx.x/blockDim.x and a
// local block index, so a role also runs alone as a per-kernel entry point.

// Router logits (8 tokens per workgroup) + Q8_K(x) + Q8_0(x).
struct PrepArgs {
  RouterLogitsArgs router;
  Q8KArgs q8k;
  Q80Args q80;
  int32_t n_router, n_q8k, n_q80;
};

// Routed gate/up/SwiGLU (IQ2_XXS) + shared gate/up/SwiGLU (Q8_0 or IQ2_XXS).
struct UpArgs {
  GateUpArgs gu;             // routed
  GateUpArgs sh_iq2;         // shared expert in IQ2_XXS (shared_fmt 1)
  Q80MatvecArgs sh_q80;      // shared expert in Q8_0 (shared_fmt 0)
  int32_t gu_tiles, gu_work; // grid = gu_tiles x gu_work
  int32_t sh_tiles, sh_work;
  int32_t sh_fmt;
  RouterSelectArgs sel;       // dsmoe_up_rows with fuse_sel: every routed workgroup runs the selection itself
  int32_t fuse_sel = 0;       // 1: the routed workgroups run the selection (T <= 8)
  // dsmoe_up_rows with fuse_midq: the workgroup that completes the 256 rows
  // of a (pair, block) writes its Q8_K (midq), the one that completes a
  // token's 256-row group of the Q8_0 shared mid writes its 8 Q8_0 blocks
  // (sh_midq); mid_cnt holds [T*k*(I/256)] routed then [T*ceil(I_s/256)]
  // shared row counters, zero between launches (each completer resets its).
  Q8KArgs midq{};
  Q80Args sh_midq{};
  uint32_t* mid_cnt = nullptr;
  int32_t fuse_midq = 0;
  int32_t sh_delay = 0;  // nonzero: the Q8_0 shared expert's workgroups start about 8 us late
};

// Q8_K of the routed mid rows (+ the IQ2 shared mid) and Q8_0 of the shared mid.
struct MidqArgs {
  Q8KArgs q8k_a;
  Q8KArgs q8k_b;
  Q80Args q80;
  int32_t n_a, n_b, n_q80;
};

// Routed down (Q2_K) + shared down (Q8_0 or Q2_K).
struct DnArgs {
  DownArgs dn;
  DownArgs sh_q2k;
  Q80MatvecArgs sh_q80;
  int32_t dn_tiles, dn_work;
  int32_t sh_tiles, sh_work;
  int32_t sh_fmt;
};

// Expert-major gate/up and down for batches with few pairs per expert: the
// pairs sorted by expert and cut into chunks of at most kEmPairs pairs of one
// expert (dsmoe_dispatch with block_m = kEmPairs); grid = max chunks x tiles.
constexpr int32_t kEmPairs = 8;  // DSMOE_EM_TILE_M
constexpr int32_t kDnEmRows = 128;  // down rows per expert-major workgroup (32 per step)
struct GuEmArgs {
  GateUpArgs gu;  // selected unused; weights per pair; mid_out [pairs][I]
  const uint32_t* sorted_pairs;
  const uint32_t* offsets;       // [E + 1]
  const uint32_t* tile_offsets;  // [E + 1]: chunks = tile_offsets[E]
  const uint32_t* tile_experts;
  const uint32_t* tile_starts;
  int32_t tiles;                 // row tiles of 32 rows
  int32_t np;                    // the dispatch's block_m (pairs per chunk), 1..kEmPairs
  // set by the forward pass when the expert-major and the grouped launches are
  // both enqueued: the workgroups return unless (*path & path_mask) == path_want
  const uint32_t* path = nullptr;
  uint32_t path_mask = 0, path_want = 0;
};
struct DnEmArgs {
  DownArgs dn;    // selected and out unused; down_out [pairs][d]
  const uint32_t* sorted_pairs;
  const uint32_t* offsets;
  const uint32_t* tile_offsets;
  const uint32_t* tile_experts;
  const uint32_t* tile_starts;
  int32_t tiles;                 // row tiles of kDnEmRows rows
  int32_t np;                    // the dispatch's block_m (pairs per chunk), 1..kEmPairs
  // set by the forward pass when the expert-major and the grouped launches are
  // both enqueued: the workgroups return unless (*path & path_mask) == path_want
  const uint32_t* path = nullptr;
  uint32_t path_mask = 0, path_want = 0;
};

// The launches of a batch with few pairs per expert on average are chosen on
// the device once the pairs are sorted (dsmoe_dispatch with a second tiling
// and path_flags): the expert-major kernels stream an expert's weights once
// per chunk of up to em_pairs pairs, the grouped ones once per 64-pair tile,
// so skewed loads (a few experts holding most pairs) go grouped.
// path_flags[0]: bit 0 gate/up grouped, bit 1 down grouped (also when
// dn_grouped: the average load alone favours it).

// Largest token count of the row-streaming (decode) launches.
constexpr int32_t kMaxDecodeT = 8;

// Grouped (sorted-by-expert) routed gate/up/SwiGLU on MFMA, for batches
// (dsmoe_gemm.hip).  A workgroup computes one tile: up to kGuBM pairs of one
// expert (a dispatch tile) x kGuBN rows of gate and of up.
struct GuGroupedArgs {
  const uint8_t* gate;            // IQ2_XXS [E][I][d/256]
  const uint8_t* up;
  const uint16_t* xh;             // Q8_K(x) qs as f16 [T][d]
  const uint8_t* xq;              // Q8_K(x) [T][d/256] (block scales)
  const uint32_t* sorted_pairs;   // [P], grouped by expert
  const uint32_t* offsets;        // [E+1] first sorted pair of each expert
  const uint32_t* tile_offsets;   // [E+1]; tile_offsets[E] = number of tiles
  const uint32_t* tile_experts;   // [tiles]
  const uint32_t* tile_starts;    // [tiles] first pair of the tile within its expert
  const float* weights;           // [P] routing weight of each pair (null: 1)
  float* mid;                     // [P][I]
  int32_t d, I, k, E;
  float clamp;
  // set by the forward pass when the expert-major and the grouped launches are
  // both enqueued: the workgroups return unless (*path & path_mask) == path_want
  const uint32_t* path = nullptr;
  uint32_t path_mask = 0, path_want = 0;
};
enum : int32_t { kGuBM = 64, kGuThreads = 512, kGuBN = kGuThreads / 2 };

// Grouped routed down projection (Q2_K) over sorted pairs: one workgroup =
// up to kGuBM pairs of one expert x kDnBN output rows; writes the per-pair
// rows (the slot sum is dsmoe_moe_sum).
struct DnGroupedArgs {
  const uint8_t* down;            // Q2_K [E][d][I/256]
  const int8_t* m8;               // Q8_K(mid) qs as int8 [P][I] (rows 16-byte aligned)
  const uint16_t* bsh;            // Q8_K(mid) bsums as f16 [P][I/16]
  const uint8_t* mq;              // Q8_K(mid) [P][I/256] (block scales)
  const uint32_t* sorted_pairs;
  const uint32_t* offsets;
  const uint32_t* tile_offsets;
  const uint32_t* tile_experts;
  const uint32_t* tile_starts;
  float* down_out;                // [P][d]
  int32_t d, I, E;
  // set by the forward pass when the expert-major and the grouped launches are
  // both enqueued: the workgroups return unless (*path & path_mask) == path_want
  const uint32_t* path = nullptr;
  uint32_t path_mask = 0, path_want = 0;
};
enum : int32_t { kDnThreads = 256, kDnBN = kDnThreads / 2 };  // 4 waves: three workgroups per CU at 168 VGPRs

// Dense Q8_0 x Q8_0-activation GEMM for batches (shared expert): tiles of
// kGuBM tokens x 64 output columns (32 gate + 32 up rows with SwiGLU, or 64
// rows of one matrix).
struct Q80GemmArgs {
  const uint8_t* w0;      // Q8_0 [out_dim][in_dim/32] (gate, or the single matrix)
  const uint8_t* w1;      // up, or null
  const uint16_t* xh;     // activation codes as f16 [T][in_dim]
  const float* xs;        // activation block scales [T][in_dim/32]
  float* out;             // [T][out_dim]: swiglu(gate, up) (weight 1), or the product
  int32_t in_dim, out_dim, T;
  float clamp;
  // split over the row's 32 lane classes (few token tiles): workgroup s of a
  // slab sums class positions [s * 32 / ksplit, (s + 1) * 32 / ksplit) into
  // part[s][T][cols] (cols = out_dim, gate then up columns with w1), and
  // dsmoe_q80_combine finishes the tree; ksplit = 1 writes out directly
  float* part = nullptr;
  int32_t ksplit = 1;
};
// dsmoe_q80_combine: out[t][c] from the ksplit partial sums (pairwise in
// split order, the top levels of the row's halving tree), then SwiGLU when
// the GEMM had two matrices.
struct Q80CombineArgs {
  const float* part;  // [ksplit][T][cols]
  float* out;         // [T][out_dim]
  int32_t out_dim, T, ksplit, two;
  float clamp;
};

// Shared expert for large batches, step 1: Q8_0 matrices rewritten in the
// operand layout of the wide GEMM (dsmoe_q80_unpack).  Row tile R (16 rows)
// and block b: codes at wh[((R * nb + b) * 64 + l) * 8 ..+8] as f16 for lane
// l = 16 q + r (row 16 R + r, codes 8 q .. 8 q + 7 of the block), and the 16
// rows' block scales as f32 at ws[(R * nb + b) * 16 ..+16].  Up to three
// matrices per launch (grid.y).
struct Q80UnpackArgs {
  const uint8_t* w[3];  // Q8_0 [rows][nb]
  uint16_t* wh[3];
  float* ws[3];
  int32_t rows[3], nb[3];
};

// Step 2: dsmoe_q80_wide / dsmoe_q80_wide_swiglu over the unpacked weights.
// Workgroup = kQwWaves waves x kQwBT tokens x kQwRows rows (kQwRowsSw row
// pairs of gate and up with SwiGLU).
struct Q80WideArgs {
  const uint16_t* w0h;  // unpacked gate (or the single matrix)
  const float* w0s;
  const uint16_t* w1h;  // unpacked up, or null
  const float* w1s;
  const uint16_t* xh;   // activation codes as f16 [T][in_dim]
  const float* xs;      // activation block scales [T][in_dim/32]
  float* out;           // [T][out_dim]
  int32_t in_dim, out_dim, T;
  float clamp;
};
#ifndef DSM_QW_WAVES
#define DSM_QW_WAVES 8
#endif
#ifndef DSM_QW_SB
#define DSM_QW_SB 2
#endif
enum { kQwWaves = DSM_QW_WAVES, kQwBT = 32 * kQwWaves, kQwRows = 16 * kQwWaves, kQwRowsSw = 8 * kQwWaves };

struct SwigluArgs {
  const float* gate;
  const float* up;
  float* out;
  int32_t n;
  float clamp, weight;
};

struct MoeSumArgs {
  const float* down;  // [T*k][d]
  float* out;         // [T][d]
  int32_t d, k, T;
};
// Four outputs per thread with 16-byte loads and stores.
inline __host__ __device__ bool moe_sum_vec_ok(const MoeSumArgs& a) {
  return a.d % 4 == 0 && (((uintptr_t)a.down | (uintptr_t)a.out) & 15) == 0;
}

// rms_norm_plain (norm.rs:14-63): one 256-thread workgroup per row.
struct RmsNormArgs {
  const float* x;
  float* out;
  int32_t n, rows;
  float eps;
};
// hc_split_weighted_sum_norm_fused (hc.rs:313-398), n_hc = 4: one 256-thread
// workgroup per row.
struct HcSplitNormArgs {
  const float* mix;          // [rows][24]
  const float* scale;        // [3]
  const float* base;         // [24]
  const float* residual_hc;  // [rows][4][n_embd]
  const float* norm_w;       // [n_embd]
  float* split;              // [rows][24]
  float* out;                // [rows][n_embd]
  float* norm_out;           // [rows][n_embd]
  int32_t n_embd, rows, iters;
  float eps, norm_eps;
};

// FFN residual merge (hc.rs:212-259): out[t][dst][i] from the layer output,
// the residual streams and the token's split row.
struct HcExpandArgs {
  const float* block_out;    // [T][n_embd]
  const float* block_add;    // [T][n_embd] (read when has_add)
  const float* residual_hc;  // [T][n_hc][n_embd]
  const float* split;        // [T][mix_hc]: pre[n_hc] | post[n_hc] | comb[n_hc][n_hc]
  float* out_hc;             // [T][n_hc][n_embd]
  int32_t n_embd, n_hc, T, mix_hc, has_add;
};
// Four outputs per thread with 16-byte accesses.
inline __host__ __device__ bool hc_expand_vec_ok(const HcExpandArgs& a) {
  return a.n_embd % 4 == 0 &&
         (((uintptr_t)a.block_out | (uintptr_t)a.residual_hc | (uintptr_t)a.out_hc |
           (a.has_add ? (uintptr_t)a.block_add : 0)) & 15) == 0;
}

struct DispatchArgs {
  const int32_t* selected;  // [pairs]
  uint32_t* counts;         // [E]
  uint32_t* offsets;        // [E+1]
  uint32_t* sorted_pairs;   // [pairs]
  uint32_t* tile_offsets;   // [E+1] or null
  uint32_t* tile_experts;   // [max tiles] or null
  uint32_t* tile_starts;    // [max tiles] or null
  int32_t pairs, E, block_m;
  // optional second tiling of the same sort (block_m2 pairs per tile) and
  // the expert-major / grouped choice from the two tile counts (ChooseArgs)
  uint32_t* tile_offsets2 = nullptr;
  uint32_t* tile_experts2 = nullptr;
  uint32_t* tile_starts2 = nullptr;
  int32_t block_m2 = 0;
  uint32_t* path_flags = nullptr;
  int32_t dn_grouped = 0;
};

// Synthetic weights: N(0, sigma) from a counter-based generator, quantized
// per 256-element superblock (or 32-element Q8_0 block, or f16/f32 element).
// Peak probes (dsmoe_probe): what this GPU sustains with no algorithm around
// it.  kind 0: dense f16 MFMA (v_mfma_f32_32x32x16_f16, eight independent
// accumulators per wave, `iters` rounds); kind 1: HBM read of `bytes` from
// `src` with 16-byte loads.  `sink` receives one float per workgroup so the
// work cannot be dropped.
struct ProbeArgs {
  const uint4* src;
  float* sink;
  uint64_t n16;   // 16-byte words of src (kind 1)
  int64_t iters;  // MFMA rounds per wave (kind 0)
};

struct SynthArgs {
  uint8_t* out;
  const uint8_t* lvlmap;  // IQ2_XXS level-tuple -> grid index map (6561 B)
  uint64_t seed;
  uint64_t tensor_id;
  int64_t n_mats;         // experts
  int32_t rows, cols;     // padded shape
  int32_t rows_real, cols_real;
  float sigma;
  int32_t fmt;            // see SynthFmt
};

enum SynthFmt : int32_t { kSynIq2xxs = 0, kSynQ2K = 1, kSynQ80 = 2, kSynF16 = 3, kSynF32 = 4 };

}  // namespace dsm
