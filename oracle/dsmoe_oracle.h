/*
 * dsmoe oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, single-source CPU restatement of the reference MoE-FFN
 * arithmetic (jbreams/deepseek-rs, engine/src/kernels/{moe,quantize,matmul,
 * utils}.rs and the call sequence in engine/src/session.rs:1894-2155).
 * It is the checker for the HIP path: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it.  The product library never
 * links or calls it.
 *
 * Every function cites the reference lines it restates.  Pinning status of
 * each function (what checks it besides the GPU) is listed in the header
 * comment of dsmoe_oracle.c.
 */
#ifndef DSMOE_ORACLE_H
#define DSMOE_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct or_config {
  int32_t d_model;      /* d, multiple of 256 */
  int32_t d_ff;         /* routed expert intermediate I, multiple of 256 */
  int32_t n_expert;     /* E */
  int32_t top_k;        /* k */
  int32_t n_group;      /* 1 = reference routing */
  int32_t topk_group;   /* groups kept when n_group > 1 */
  float route_scale;    /* 1.5 in the reference */
  float swiglu_clamp;   /* 10.0 in the reference */
  int32_t has_bias;
  int32_t shared_fmt;   /* 0 = Q8_0 (reference), 1 = IQ2_XXS/Q2_K, -1 = none */
  int32_t d_ff_shared;  /* shared expert intermediate */
} or_config;

float or_f16_to_f32(uint16_t h);
float or_expf(float x);
float or_logf(float y);
float or_softplus(float x);
float or_silu(float g);
uint8_t or_iq2_sign(uint32_t idx7);
uint64_t or_iq2_grid(uint32_t idx);

/* block dots */
float or_dot_iq2_xxs_q8k(const uint8_t* iq2, const uint8_t* q8k);
int32_t or_iq2_xxs_bsum(const uint8_t* iq2, const uint8_t* q8k);
float or_dot_q2k_q8k(const uint8_t* q2k, const uint8_t* q8k);
void or_q2k_isum_summs(const uint8_t* q2k, const uint8_t* q8k, int32_t* isum, int32_t* summs);

/* activation quantizers */
void or_q8k_quantize(const float* x, uint8_t* out, int in_dim, int rows);
void or_q8_0_quantize(const float* x, int8_t* xq, float* xscale, int in_dim, int rows);

/* dense pieces */
void or_router_logits(const uint16_t* w, const float* x, float* out, int d, int E, int T, int nthreads);
void or_router_select_hash(const or_config* c, const float* logits, const int32_t* hash, int hash_rows,
                           const int32_t* tokens, int token_scalar, int T, float* probs, int32_t* selected,
                           float* weights);
void or_router_select(const or_config* c, const float* logits, const float* bias, int T,
                      float* probs, int32_t* selected, float* weights);
void or_q8_0_matvec(const uint8_t* w, const int8_t* xq, const float* xscale, float* out,
                    int in_dim, int out_dim, int T, int nthreads);
void or_swiglu(const float* gate, const float* up, float* out, int n, float clamp, float weight);

/* routed experts */
void or_gate_up_mid(const uint8_t* gate, const uint8_t* up, const uint8_t* xq,
                    const int32_t* selected, const float* weights,
                    float* gate_out, float* up_out, float* mid_out,
                    int d, int I, int T, int k, float clamp, int nthreads);
void or_down(const uint8_t* down, const uint8_t* midq, const int32_t* selected,
             float* down_out, int d, int I, int T, int k, int nthreads);
void or_moe_sum(const float* down, float* out, int d, int k, int T);
void or_rms_norm_plain(const float* x, float* out, int n, int rows, float eps);
void or_hc4_split(const float* mix, const float* scale, const float* base, int iters, float eps, float* out);
void or_hc_split_norm(const float* mix, const float* scale, const float* base, const float* residual_hc,
                      const float* norm_w, float* split, float* out, float* norm_out, int n_embd, int n_rows,
                      int iters, float eps, float norm_eps);
void or_hc_expand(const float* block_out, const float* block_add, const float* residual_hc, const float* split,
                  float* out_hc, int n_embd, int n_hc, int n_tokens, int mix_hc, int has_add);

/* dispatch */
void or_dispatch(const int32_t* selected, int pairs, int E, int block_m,
                 uint32_t* counts, uint32_t* offsets, uint32_t* sorted_pairs,
                 uint32_t* tile_offsets, uint32_t* tile_experts, uint32_t* tile_starts);

/* whole layer: shared_out[T,d], routed_out[T,d]; selected/weights [T,k] may be NULL */
int or_moe_forward(const or_config* c,
                   const uint16_t* w_router, const float* bias,
                   const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                   const uint8_t* w_sh_gate, const uint8_t* w_sh_up, const uint8_t* w_sh_down,
                   const float* x, int T, float* shared_out, float* routed_out,
                   int32_t* selected, float* weights, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
