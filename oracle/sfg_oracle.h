/*
 * sfg_oracle.h -- CPU restatement of SchedForge's decoder-layer execution path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP backend:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * The product (schedforge_amd/, libsfg_hip.so) never links, loads or calls it.
 *
 * Every function restates one reference function; the citation is given at the
 * definition in sfg_oracle.c (paths relative to the reference repository root).
 * Arithmetic follows the reference: fp32 values, sequential-k fp32 FMA chains for
 * matrix products (what g++ -march=native emits for the reference's scalar loops),
 * RMSNorm sum of squares in double, weight-only int8 with fp32 activations.
 *
 * Parity pins (tests/test_oracle.py): closed forms (RMSNorm of a constant row,
 * RoPE at position 0 / pair-norm preservation, attention with equal keys and
 * one-hot values), brute-force fp64 restatements at tiny shapes, integer-exact
 * GEMMs, the reference's own known-answer tests (paged gather of iota inputs,
 * constant int8 matmul, bf16 conversion values, routing invariants) and the
 * committed golden vectors under tests/golden/.
 */
#ifndef SFG_ORACLE_H
#define SFG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synthetic inputs: counter-based N(mean, std) keyed by (seed, tensor, index) ---- */
uint64_t sfgo_splitmix64(uint64_t x);
void sfgo_fill_normal(uint64_t seed, uint32_t tensor_id, float mean, float stddev,
                      float* out, int64_t count);
void sfgo_page_permutation(uint64_t seed, int32_t* perm, int64_t count);

/* ---- bf16 (compiler.cpp:34-52) ---- */
void sfgo_to_bf16(const float* in, uint16_t* out, int64_t count);
void sfgo_from_bf16(const uint16_t* in, float* out, int64_t count);
void sfgo_round_bf16(float* values, int64_t count);

/* ---- dense building blocks ---- */
void sfgo_rms_norm(const float* x, const float* w, float* y, int64_t rows, int64_t width,
                   float eps);
void sfgo_matmul(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k);
void sfgo_concat_columns(const float* const* weights, const int64_t* widths, int64_t count,
                         int64_t input_width, float* packed);
void sfgo_rope_at(float* t, int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                  float theta, int64_t pos0);
void sfgo_rope(float* t, int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
               float theta);
void sfgo_split_qkv_rope(const float* qkv, int64_t batch, int64_t seq, int64_t hidden,
                         int64_t q_heads, int64_t kv_heads, int64_t head_dim, float theta,
                         float* q, float* k, float* v);
void sfgo_merge_heads(const float* attn, int64_t batch, int64_t seq, int64_t heads,
                      int64_t head_dim, float* merged);
void sfgo_swiglu(const float* gate_up, int64_t rows, int64_t inter, float* out);
void sfgo_add(const float* a, const float* b, float* out, int64_t count);

typedef struct {
    int32_t batch, query_heads, kv_heads, seq_q, seq_kv, head_dim, head_dim_value;
    int32_t causal;
    float scale; /* <= 0: 1/sqrt(head_dim) */
} sfgo_attn_cfg;
void sfgo_attention(const sfgo_attn_cfg* cfg, const float* q, const float* k, const float* v,
                    float* out);

/* ---- paged KV (next_milestones.cpp) and the build's per-sequence page tables ---- */
void sfgo_paged_gather(const float* pool, const int32_t* page_table, int64_t batch,
                       int64_t kv_heads, int64_t ctx, int64_t page_tokens, int64_t head_dim,
                       int64_t pages_per_seq, float* flat);
void sfgo_paged_scatter(const float* flat, const int32_t* page_table, int64_t batch,
                        int64_t kv_heads, int64_t ctx, int64_t page_tokens, int64_t head_dim,
                        int64_t pages_per_seq, float* pool);

/* ---- MoE ---- */
void sfgo_route_topk(const float* x, const float* router, const float* bias, int64_t tokens,
                     int64_t hidden, int64_t experts, int64_t top_k, int32_t* ids,
                     float* weights, int32_t* counts);
void sfgo_dispatch(const int32_t* ids, const float* weights, const int32_t* counts,
                   int64_t tokens, int64_t experts, int64_t top_k, int32_t* offsets,
                   int32_t* token_ids, int32_t* route_slots, float* routing_weights);
void sfgo_moe_reference(const float* x, const float* w1, const float* w3, const float* w2,
                        int64_t tokens, int64_t hidden, int64_t inter, int64_t top_k,
                        const int32_t* ids, const float* weights, float* out);

/* ---- weight-only int8 (next_milestones.cpp) ---- */
void sfgo_transpose(const float* in, int64_t rows, int64_t cols, float* out);
void sfgo_quantize_nk(const float* w_nk, int64_t n, int64_t k, int8_t* q, float* scales);
void sfgo_quantized_matmul(const float* x, const int8_t* q_nk, const float* scales,
                           int64_t m, int64_t n, int64_t k, float* out);
void sfgo_quantized_moe(const float* x, const int8_t* w1q, const float* s1,
                        const int8_t* w3q, const float* s3, const int8_t* w2q,
                        const float* s2, int64_t tokens, int64_t hidden, int64_t inter,
                        int64_t top_k, const int32_t* ids, const float* weights, float* out);

/* ---- whole layer (decoder_compiler.cpp:622-673 + next_milestones.cpp composition) ---- */
typedef struct {
    int32_t batch, sequence, hidden, intermediate, query_heads, kv_heads, head_dim;
    float rms_epsilon, rope_theta;
    int32_t causal;
    int32_t moe;          /* 0 dense SwiGLU, 1 MoE */
    int32_t experts, top_k;
    int32_t context;      /* 0 prefill, >0 decode over cached K/V of this length */
    int32_t int8_weights; /* 1: projections and FFN weights are weight-only int8 */
    int32_t threads;      /* OpenMP threads for the oracle (<=0: default) */
    int32_t kv_append;    /* decode: 1 = the build's append mode (true-position RoPE, the
                             step's K/V appended to the cache and attended over) */
    int32_t kv_pool_f32;  /* append mode: the pools hold fp32 (the fp32 path), so the
                             appended K/V keep fp32; 0: bf16 pools, rounded to bf16 */
} sfgo_layer_cfg;

typedef struct {
    const float* input;                 /* [rows, H] */
    const float* rms1;                  /* [H] */
    const float* wq; const float* wk; const float* wv; /* [H, H], [H, kvD], [H, kvD] */
    const float* wo;                    /* [H, H] */
    const float* rms2;                  /* [H] */
    const float* wg; const float* wu;   /* [H, I] */
    const float* wd;                    /* [I, H] */
    const float* router;                /* [H, E] */
    const float* router_bias;           /* [E] or NULL */
    const float* w1; const float* w3;   /* [E, H, I] */
    const float* w2;                    /* [E, I, H] */
    const float* cached_k; const float* cached_v; /* [B, Hkv, ctx, D] */
    const int32_t* trace_ids;           /* optional routing trace [rows, k] */
    const float* trace_weights;
    /* int8 mode: quantized [N][K] weights + per-channel scales (q,k,v,o,g,u,d) */
    const int8_t* q8[7]; const float* s8[7];
    const int8_t* e1q; const float* e1s; /* [E][I][H], [E][I] */
    const int8_t* e3q; const float* e3s;
    const int8_t* e2q; const float* e2s; /* [E][H][I], [E][H] */
} sfgo_layer_data;

typedef struct {  /* optional intermediates for stage-level checks (each may be NULL) */
    float* normalized1;  /* [rows, H] */
    float* qkv;          /* [rows, H + 2 kvD] */
    float* attn_merged;  /* [rows, H] */
    float* residual1;    /* [rows, H] */
    float* normalized2;  /* [rows, H] */
    int32_t* ids; float* weights; int32_t* counts; /* routing */
    float* new_k; float* new_v;  /* append mode: the step's K/V as stored [B,Hkv,S,D] */
} sfgo_layer_taps;

int sfgo_decoder_layer(const sfgo_layer_cfg* cfg, const sfgo_layer_data* d, float* out,
                       sfgo_layer_taps* taps);
/* Prefill layer at the rows sample[0..n) only (row = b * S + s): out [n][H] and
 * n-row taps equal those rows of sfgo_decoder_layer bit for bit. */
int sfgo_decoder_layer_rows(const sfgo_layer_cfg* cfg, const sfgo_layer_data* d,
                            const int64_t* sample, int64_t n, float* out, sfgo_layer_taps* taps);

double sfgo_max_abs_error(const float* a, const float* b, int64_t count);
int sfgo_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
