/*
 * sfg_oracle.c -- CPU restatement of SchedForge's decoder-layer path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP backend.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Reference citations are file:line in the SchedForge repository.  Where the
 * reference leaves bits to its compiler (FMA contraction under -march=native),
 * this file spells the FMA out with fmaf() and is compiled with
 * -ffp-contract=off so every other expression rounds exactly as written.
 *
 * Parity status per function is listed in the header comment of
 * tests/test_oracle.py next to the check that pins it.
 */
#include "sfg_oracle.h"

#include <float.h>
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define IDX(type, x) ((type)(x))

int sfgo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------- */
/* Synthetic inputs (build-side spec; the reference's own generators use     */
/* std::mt19937 + uniform_real_distribution, decoder_compiler.cpp:483-514,    */
/* whose bits depend on the C++ library, so they are not reused).             */
/* ------------------------------------------------------------------------- */

uint64_t sfgo_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static uint64_t stream_key(uint64_t seed, uint32_t tensor_id) {
    return sfgo_splitmix64(sfgo_splitmix64(seed) ^ ((uint64_t)tensor_id * 0xD1B54A32D192ED03ULL));
}

/* Element i of tensor `tensor_id`: Box-Muller (cosine branch) in double on two
 * 53-bit uniforms drawn from the counter stream at 2i and 2i+1. */
void sfgo_fill_normal(uint64_t seed, uint32_t tensor_id, float mean, float stddev,
                      float* out, int64_t count) {
    const uint64_t key = stream_key(seed, tensor_id);
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        const uint64_t r1 = sfgo_splitmix64(key + 2 * (uint64_t)i);
        const uint64_t r2 = sfgo_splitmix64(key + 2 * (uint64_t)i + 1);
        const double u1 = ((double)(r1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
        const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = (float)((double)mean + (double)stddev * z);
    }
}

/* Seeded Fisher-Yates permutation of 0..count-1 (physical page assignment). */
void sfgo_page_permutation(uint64_t seed, int32_t* perm, int64_t count) {
    const uint64_t key = stream_key(seed, 17u);
    for (int64_t i = 0; i < count; ++i) perm[i] = (int32_t)i;
    for (int64_t i = count - 1; i > 0; --i) {
        const uint64_t r = sfgo_splitmix64(key + (uint64_t)i);
        const int64_t j = (int64_t)(r % (uint64_t)(i + 1));
        const int32_t t = perm[i];
        perm[i] = perm[j];
        perm[j] = t;
    }
}

/* ------------------------------------------------------------------------- */
/* bf16: convert_to_bf16 / convert_from_bf16 (compiler.cpp:34-52).            */
/* Round to nearest even by adding 0x7FFF + lsb, no NaN special case.         */
/* ------------------------------------------------------------------------- */

void sfgo_to_bf16(const float* in, uint16_t* out, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        uint32_t bits;
        memcpy(&bits, &in[i], sizeof bits);
        const uint32_t rounding = 0x7FFFu + ((bits >> 16) & 1u);
        out[i] = (uint16_t)((bits + rounding) >> 16);
    }
}

void sfgo_from_bf16(const uint16_t* in, float* out, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        const uint32_t bits = (uint32_t)in[i] << 16;
        memcpy(&out[i], &bits, sizeof bits);
    }
}

void sfgo_round_bf16(float* values, int64_t count) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        uint32_t bits;
        memcpy(&bits, &values[i], sizeof bits);
        const uint32_t rounding = 0x7FFFu + ((bits >> 16) & 1u);
        bits = ((bits + rounding) >> 16) << 16;
        memcpy(&values[i], &bits, sizeof bits);
    }
}

/* ------------------------------------------------------------------------- */
/* Dense building blocks                                                      */
/* ------------------------------------------------------------------------- */

/* rms_norm (decoder_compiler.cpp:41-62): sum of squares in double, inverse
 * 1/sqrtf(float(sum/width) + eps) in float, y = (x * inv) * w. */
void sfgo_rms_norm(const float* x, const float* w, float* y, int64_t rows, int64_t width,
                   float eps) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * width;
        double sum = 0.0;
        for (int64_t c = 0; c < width; ++c) sum += (double)xr[c] * (double)xr[c];
        const float inv = 1.0f / sqrtf((float)(sum / (double)width) + eps);
        for (int64_t c = 0; c < width; ++c) y[r * width + c] = xr[c] * inv * w[c];
    }
}

/* scalar_matmul (decoder_compiler.cpp:64-75) and the register kernels of
 * execute(LoopIR) (runtime.cpp:278-438): every output is a sequential fp32 FMA
 * chain over k starting from 0.
 *
 * Blocking keeps that chain.  Work is cut into tiles of MM_TM rows x MM_TN
 * columns (the OpenMP tasks), each walked in k blocks of MM_TK.  Inside a
 * block a 4 x 32 register kernel holds sixteen 8-lane accumulators, one lane
 * per output, and adds one rounded fused product per k in increasing order;
 * the accumulators go back to c between k blocks and resume from there.
 * Storing and reloading an fp32 value is exact, and _mm256_fmadd_ps is the
 * lane-wise fmaf, so every output gets the same rounding sequence as the
 * plain i-k-j loop -- which is what the remainder rows and columns run. */
#define MM_TM 64
#define MM_TN 256
#define MM_TK 256

/* c[0:4][0:32] (row stride ldc) over kn steps: row r of a (stride lda) and a
 * packed B panel bp [kn][32], both starting at the block's first k; first:
 * start the chains from 0. */
static void mm_kernel_4x32(const float* a, int64_t lda, const float* bp, float* c, int64_t ldc,
                           int64_t kn, int first) {
    __m256 acc[4][4];
    for (int r = 0; r < 4; ++r)
        for (int v = 0; v < 4; ++v)
            acc[r][v] = first ? _mm256_setzero_ps() : _mm256_loadu_ps(c + r * ldc + 8 * v);
    for (int64_t t = 0; t < kn; ++t) {
        const float* br = bp + t * 32;
        const __m256 b0 = _mm256_loadu_ps(br), b1 = _mm256_loadu_ps(br + 8);
        const __m256 b2 = _mm256_loadu_ps(br + 16), b3 = _mm256_loadu_ps(br + 24);
        for (int r = 0; r < 4; ++r) {
            const __m256 ar = _mm256_broadcast_ss(a + r * lda + t);
            acc[r][0] = _mm256_fmadd_ps(ar, b0, acc[r][0]);
            acc[r][1] = _mm256_fmadd_ps(ar, b1, acc[r][1]);
            acc[r][2] = _mm256_fmadd_ps(ar, b2, acc[r][2]);
            acc[r][3] = _mm256_fmadd_ps(ar, b3, acc[r][3]);
        }
    }
    for (int r = 0; r < 4; ++r)
        for (int v = 0; v < 4; ++v) _mm256_storeu_ps(c + r * ldc + 8 * v, acc[r][v]);
}

/* The plain chain for outputs [i0,i1) x [j0,j1) over k in [k0, k1). */
static void mm_edge(const float* a, const float* b, float* c, int64_t n, int64_t k, int64_t i0,
                    int64_t i1, int64_t j0, int64_t j1, int64_t k0, int64_t k1) {
    for (int64_t i = i0; i < i1; ++i) {
        float* crow = c + i * n;
        if (k0 == 0)
            for (int64_t j = j0; j < j1; ++j) crow[j] = 0.0f;
        for (int64_t kk = k0; kk < k1; ++kk) {
            const float aik = a[i * k + kk];
            const float* brow = b + kk * n;
            for (int64_t j = j0; j < j1; ++j) crow[j] = fmaf(aik, brow[j], crow[j]);
        }
    }
}

void sfgo_matmul(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k) {
    const int64_t tiles_m = (m + MM_TM - 1) / MM_TM, tiles_n = (n + MM_TN - 1) / MM_TN;
    if (k <= 0) {
        for (int64_t i = 0; i < m * n; ++i) c[i] = 0.0f;
        return;
    }
#pragma omp parallel
    {
        /* this thread's packed copy of one B block: MM_TN / 32 panels [MM_TK][32] */
        float* bp = (float*)malloc(sizeof(float) * MM_TK * MM_TN);
#pragma omp for schedule(dynamic, 1)
        for (int64_t t = 0; t < tiles_m * tiles_n; ++t) {
            /* column tiles outermost: neighbouring tasks share a B panel */
            const int64_t i0 = (t % tiles_m) * MM_TM, j0 = (t / tiles_m) * MM_TN;
            const int64_t i1 = i0 + MM_TM < m ? i0 + MM_TM : m;
            const int64_t j1 = j0 + MM_TN < n ? j0 + MM_TN : n;
            const int64_t i4 = i0 + (i1 - i0) / 4 * 4, j32 = j0 + (j1 - j0) / 32 * 32;
            for (int64_t k0 = 0; k0 < k; k0 += MM_TK) {
                const int64_t k1 = k0 + MM_TK < k ? k0 + MM_TK : k, kn = k1 - k0;
                if (i4 > i0)
                    for (int64_t j = j0; j < j32; j += 32) {
                        float* panel = bp + (j - j0) * MM_TK;
                        for (int64_t kk = k0; kk < k1; ++kk)
                            memcpy(panel + (kk - k0) * 32, b + kk * n + j, 32 * sizeof(float));
                        for (int64_t i = i0; i < i4; i += 4)
                            mm_kernel_4x32(a + i * k + k0, k, panel, c + i * n + j, n, kn, k0 == 0);
                    }
                if (j32 < j1) mm_edge(a, b, c, n, k, i0, i4, j32, j1, k0, k1);
                if (i4 < i1) mm_edge(a, b, c, n, k, i4, i1, j0, j1, k0, k1);
            }
        }
        free(bp);
    }
}

/* concatenate_columns (decoder_compiler.cpp:77-94). */
void sfgo_concat_columns(const float* const* weights, const int64_t* widths, int64_t count,
                         int64_t input_width, float* packed) {
    int64_t total = 0;
    for (int64_t t = 0; t < count; ++t) total += widths[t];
    for (int64_t r = 0; r < input_width; ++r) {
        int64_t dst = 0;
        for (int64_t t = 0; t < count; ++t) {
            memcpy(packed + r * total + dst, weights[t] + r * widths[t],
                   (size_t)widths[t] * sizeof(float));
            dst += widths[t];
        }
    }
}

/* apply_rope (decoder_compiler.cpp:96-114): interleaved pairs (2i, 2i+1),
 * f = powf(theta, -(2i)/D), angle = float(pos) * f, pos = index within seq. */
void sfgo_rope(float* t, int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
               float theta) {
    sfgo_rope_at(t, batch, heads, seq, head_dim, theta, 0);
}

/* The same rotation with token s at position pos0 + s: the build's append mode
 * rotates a decode step's token at its true position (the reference always uses
 * the index within the step, decoder_compiler.cpp:96-104). */
void sfgo_rope_at(float* t, int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                  float theta, int64_t pos0) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t s = 0; s < seq; ++s)
                for (int64_t d = 0; d + 1 < head_dim; d += 2) {
                    const float freq = powf(theta, -(float)d / (float)head_dim);
                    const float angle = (float)(pos0 + s) * freq;
                    const float cs = cosf(angle);
                    const float sn = sinf(angle);
                    float* base = t + (((b * heads + h) * seq + s) * head_dim + d);
                    const float even = base[0];
                    const float odd = base[1];
                    base[0] = even * cs - odd * sn;
                    base[1] = even * sn + odd * cs;
                }
}

/* split_qkv (decoder_compiler.cpp:116-148): [rows, H + 2 kvD] -> Q [B,Hq,S,D],
 * K, V [B,Hkv,S,D]; RoPE on Q and K. */
void sfgo_split_qkv_rope(const float* qkv, int64_t batch, int64_t seq, int64_t hidden,
                         int64_t q_heads, int64_t kv_heads, int64_t head_dim, float theta,
                         float* q, float* k, float* v) {
    const int64_t kv = kv_heads * head_dim;
    const int64_t total = hidden + 2 * kv;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t s = 0; s < seq; ++s) {
            const float* row = qkv + (b * seq + s) * total;
            for (int64_t h = 0; h < q_heads; ++h)
                for (int64_t d = 0; d < head_dim; ++d)
                    q[((b * q_heads + h) * seq + s) * head_dim + d] = row[h * head_dim + d];
            for (int64_t h = 0; h < kv_heads; ++h)
                for (int64_t d = 0; d < head_dim; ++d) {
                    const int64_t dst = ((b * kv_heads + h) * seq + s) * head_dim + d;
                    k[dst] = row[hidden + h * head_dim + d];
                    v[dst] = row[hidden + kv + h * head_dim + d];
                }
        }
    sfgo_rope(q, batch, q_heads, seq, head_dim, theta);
    sfgo_rope(k, batch, kv_heads, seq, head_dim, theta);
}

/* merge_attention (decoder_compiler.cpp:150-174): head-major -> [rows, H]. */
void sfgo_merge_heads(const float* attn, int64_t batch, int64_t seq, int64_t heads,
                      int64_t head_dim, float* merged) {
    const int64_t hidden = heads * head_dim;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t s = 0; s < seq; ++s)
                for (int64_t d = 0; d < head_dim; ++d)
                    merged[(b * seq + s) * hidden + h * head_dim + d] =
                        attn[((b * heads + h) * seq + s) * head_dim + d];
}

/* swiglu (decoder_compiler.cpp:183-194): silu(gate) * up, gate = first I columns. */
void sfgo_swiglu(const float* gate_up, int64_t rows, int64_t inter, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < inter; ++c) {
            const float g = gate_up[r * 2 * inter + c];
            const float u = gate_up[r * 2 * inter + inter + c];
            out[r * inter + c] = g / (1.0f + expf(-g)) * u;
        }
}

/* add (decoder_compiler.cpp:176-181). */
void sfgo_add(const float* a, const float* b, float* out, int64_t count) {
    for (int64_t i = 0; i < count; ++i) out[i] = a[i] + b[i];
}

/* reference_attention (attention_compiler.cpp:742-781): two-pass softmax per
 * (batch, head, query); causal alignment j <= Skv - Sq + i (68-72); GQA
 * kv_head = h * Hkv / Hq; scale 1/sqrt(D) unless cfg->scale > 0 (43-46). */
/* One query row: qr [D] against keys / values kb, vb ([seq_kv][D], [seq_kv][Dv]
 * of its kv head) up to key `limit`; scores is scratch of seq_kv floats. */
static void attention_row(const float* qr, const float* kb, const float* vb, int64_t seq_kv,
                          int64_t limit, int64_t D, int64_t Dv, float scale, float* scores,
                          float* orow) {
    float maximum = -INFINITY;
    const int64_t count = limit + 1 < seq_kv ? limit + 1 : seq_kv;
    int64_t j = 0;
    /* eight keys at a time: eight independent dot chains, each still summed
     * over d in order (the same bits as one key at a time) */
    for (; j + 8 <= count; j += 8) {
        float dot[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        const float* kr = kb + j * D;
        for (int64_t d = 0; d < D; ++d) {
            const float qd = qr[d];
            for (int t = 0; t < 8; ++t) dot[t] = fmaf(qd, kr[t * D + d], dot[t]);
        }
        for (int t = 0; t < 8; ++t) {
            scores[j + t] = dot[t] * scale;
            if (scores[j + t] > maximum) maximum = scores[j + t];
        }
    }
    for (; j < count; ++j) {
        const float* kr = kb + j * D;
        float dot = 0.0f;
        for (int64_t d = 0; d < D; ++d) dot = fmaf(qr[d], kr[d], dot);
        scores[j] = dot * scale;
        if (scores[j] > maximum) maximum = scores[j];
    }
    for (int64_t d = 0; d < Dv; ++d) orow[d] = 0.0f;
    float denom = 0.0f;
    for (int64_t j = 0; j <= limit && j < seq_kv; ++j) {
        const float p = expf(scores[j] - maximum);
        denom += p;
        const float* vr = vb + j * Dv;
        for (int64_t d = 0; d < Dv; ++d) orow[d] = fmaf(p, vr[d], orow[d]);
    }
    for (int64_t d = 0; d < Dv; ++d) orow[d] /= denom;
}

static float attention_scale(const sfgo_attn_cfg* c) {
    return c->scale > 0.0f ? c->scale : 1.0f / sqrtf((float)c->head_dim);
}

void sfgo_attention(const sfgo_attn_cfg* c, const float* q, const float* k, const float* v,
                    float* out) {
    const float scale = attention_scale(c);
    const int64_t D = c->head_dim, Dv = c->head_dim_value;
    const int64_t pairs = (int64_t)c->batch * c->query_heads;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t bh = 0; bh < pairs; ++bh) {
        const int64_t b = bh / c->query_heads, h = bh % c->query_heads;
        const int64_t kvh = h * c->kv_heads / c->query_heads;
        float* scores = (float*)malloc(sizeof(float) * (size_t)c->seq_kv);
        const float* kb = k + (b * c->kv_heads + kvh) * c->seq_kv * D;
        const float* vb = v + (b * c->kv_heads + kvh) * c->seq_kv * Dv;
        for (int64_t i = 0; i < c->seq_q; ++i) {
            const int64_t limit = c->causal ? (c->seq_kv - c->seq_q + i) : (c->seq_kv - 1);
            attention_row(q + ((b * c->query_heads + h) * c->seq_q + i) * D, kb, vb, c->seq_kv,
                          limit, D, Dv, scale, scores,
                          out + ((b * c->query_heads + h) * c->seq_q + i) * Dv);
        }
        free(scores);
    }
}

/* ------------------------------------------------------------------------- */
/* Paged KV.  The reference pool is [page][B][Hkv][page_tok][D] with one      */
/* table shared by the batch (next_milestones.cpp:29-33, 122-129,              */
/* gather_paged_kv 560-581).  The build stores [page][Hkv][page_tok][D] with  */
/* a table per sequence; gather maps both to [B, Hkv, ctx, D].                */
/* ------------------------------------------------------------------------- */

void sfgo_paged_gather(const float* pool, const int32_t* page_table, int64_t batch,
                       int64_t kv_heads, int64_t ctx, int64_t page_tokens, int64_t head_dim,
                       int64_t pages_per_seq, float* flat) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < kv_heads; ++h)
            for (int64_t t = 0; t < ctx; ++t) {
                const int64_t page = page_table[b * pages_per_seq + t / page_tokens];
                const float* src = pool + ((page * kv_heads + h) * page_tokens + t % page_tokens) *
                                              head_dim;
                memcpy(flat + ((b * kv_heads + h) * ctx + t) * head_dim, src,
                       (size_t)head_dim * sizeof(float));
            }
}

void sfgo_paged_scatter(const float* flat, const int32_t* page_table, int64_t batch,
                        int64_t kv_heads, int64_t ctx, int64_t page_tokens, int64_t head_dim,
                        int64_t pages_per_seq, float* pool) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < kv_heads; ++h)
            for (int64_t t = 0; t < ctx; ++t) {
                const int64_t page = page_table[b * pages_per_seq + t / page_tokens];
                float* dst = pool + ((page * kv_heads + h) * page_tokens + t % page_tokens) *
                                        head_dim;
                memcpy(dst, flat + ((b * kv_heads + h) * ctx + t) * head_dim,
                       (size_t)head_dim * sizeof(float));
            }
}

/* ------------------------------------------------------------------------- */
/* MoE                                                                        */
/* ------------------------------------------------------------------------- */

/* route_topk (moe_compiler.cpp:412-455): logits as a sequential fp32 FMA chain
 * over features; optional per-expert bias added to the logit (build extension
 * for the skewed-load config); softmax over all experts, max-shifted; top-k by
 * probability with slot 0 the largest; weights renormalised over the selected
 * experts.  Selection compares logits (softmax is strictly monotone, so this is
 * the probability order) and breaks ties toward the lower expert index. */
void sfgo_route_topk(const float* x, const float* router, const float* bias, int64_t tokens,
                     int64_t hidden, int64_t experts, int64_t top_k, int32_t* ids,
                     float* weights, int32_t* counts) {
    for (int64_t e = 0; e < experts; ++e) counts[e] = 0;
    float* logits = (float*)malloc(sizeof(float) * (size_t)experts);
    float* probs = (float*)malloc(sizeof(float) * (size_t)experts);
    int32_t* taken = (int32_t*)malloc(sizeof(int32_t) * (size_t)experts);
    for (int64_t t = 0; t < tokens; ++t) {
        float maximum = -INFINITY;
        for (int64_t e = 0; e < experts; ++e) {
            float value = 0.0f;
            for (int64_t f = 0; f < hidden; ++f)
                value = fmaf(x[t * hidden + f], router[f * experts + e], value);
            if (bias) value = value + bias[e];
            logits[e] = value;
            if (value > maximum) maximum = value;
            taken[e] = 0;
        }
        float denom = 0.0f;
        for (int64_t e = 0; e < experts; ++e) {
            probs[e] = expf(logits[e] - maximum);
            denom += probs[e];
        }
        float selected = 0.0f;
        for (int64_t s = 0; s < top_k; ++s) {
            int64_t best = -1;
            for (int64_t e = 0; e < experts; ++e) {
                if (taken[e]) continue;
                if (best < 0 || logits[e] > logits[best]) best = e;
            }
            taken[best] = 1;
            ids[t * top_k + s] = (int32_t)best;
            selected += probs[best] / denom;
        }
        for (int64_t s = 0; s < top_k; ++s) {
            const int32_t e = ids[t * top_k + s];
            weights[t * top_k + s] = (probs[e] / denom) / selected;
            counts[e] += 1;
        }
    }
    free(logits);
    free(probs);
    free(taken);
}

/* dispatch_tokens (moe_compiler.cpp:496-528): offsets = exclusive prefix of
 * counts (E+1 entries); assignments visited token-ascending, slot-ascending,
 * each placed at cursor[expert]++ (a stable sort by expert). */
void sfgo_dispatch(const int32_t* ids, const float* weights, const int32_t* counts,
                   int64_t tokens, int64_t experts, int64_t top_k, int32_t* offsets,
                   int32_t* token_ids, int32_t* route_slots, float* routing_weights) {
    offsets[0] = 0;
    for (int64_t e = 0; e < experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)(experts + 1));
    memcpy(cursor, offsets, sizeof(int32_t) * (size_t)(experts + 1));
    for (int64_t t = 0; t < tokens; ++t)
        for (int64_t s = 0; s < top_k; ++s) {
            const int32_t e = ids[t * top_k + s];
            const int32_t dst = cursor[e]++;
            token_ids[dst] = (int32_t)t;
            route_slots[dst] = (int32_t)s;
            routing_weights[dst] = weights[t * top_k + s];
        }
    free(cursor);
}

/* reference_moe (moe_compiler.cpp:640-682): per token and slot,
 * gate = x W1[e], up = silu(x W3[e]) (silu on W3), y += w * ((gate*up) W2[e]).
 * Token rows routed to one expert are batched so the products vectorise; each
 * output element is still a sequential FMA chain in the reference's order. */
void sfgo_moe_reference(const float* x, const float* w1, const float* w3, const float* w2,
                        int64_t tokens, int64_t hidden, int64_t inter, int64_t top_k,
                        const int32_t* ids, const float* weights, float* out) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < tokens; ++t) {
        float* first = (float*)malloc(sizeof(float) * (size_t)inter);
        float* third = (float*)malloc(sizeof(float) * (size_t)inter);
        float* y = (float*)malloc(sizeof(float) * (size_t)hidden);
        float* orow = out + t * hidden;
        for (int64_t f = 0; f < hidden; ++f) orow[f] = 0.0f;
        for (int64_t s = 0; s < top_k; ++s) {
            const int64_t e = ids[t * top_k + s];
            const float w = weights[t * top_k + s];
            const float* e1 = w1 + e * hidden * inter;
            const float* e3 = w3 + e * hidden * inter;
            const float* e2 = w2 + e * inter * hidden;
            for (int64_t i = 0; i < inter; ++i) { first[i] = 0.0f; third[i] = 0.0f; }
            for (int64_t f = 0; f < hidden; ++f) {
                const float xv = x[t * hidden + f];
                const float* r1 = e1 + f * inter;
                const float* r3 = e3 + f * inter;
                for (int64_t i = 0; i < inter; ++i) {
                    first[i] = fmaf(xv, r1[i], first[i]);
                    third[i] = fmaf(xv, r3[i], third[i]);
                }
            }
            for (int64_t i = 0; i < inter; ++i)
                first[i] = first[i] * (third[i] / (1.0f + expf(-third[i])));
            for (int64_t f = 0; f < hidden; ++f) y[f] = 0.0f;
            for (int64_t i = 0; i < inter; ++i) {
                const float a = first[i];
                const float* r2 = e2 + i * hidden;
                for (int64_t f = 0; f < hidden; ++f) y[f] = fmaf(a, r2[f], y[f]);
            }
            for (int64_t f = 0; f < hidden; ++f) orow[f] = fmaf(w, y[f], orow[f]);
        }
        free(first);
        free(third);
        free(y);
    }
}

/* ------------------------------------------------------------------------- */
/* Weight-only int8                                                           */
/* ------------------------------------------------------------------------- */

/* transpose_decoder_weight (next_milestones.cpp:233-244): [K,N] -> [N,K]. */
void sfgo_transpose(const float* in, int64_t rows, int64_t cols, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) out[c * rows + r] = in[r * cols + c];
}

/* quantize_matmul_weights (next_milestones.cpp:611-637), per channel:
 * s_n = max_k |w| / 127 (1 when the column is all zero), q = clamp(round(w/s))
 * with round half away from zero, zero point 0, storage [N][K]. */
void sfgo_quantize_nk(const float* w_nk, int64_t n, int64_t k, int8_t* q, float* scales) {
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < n; ++c) {
        float maximum = 0.0f;
        for (int64_t d = 0; d < k; ++d) {
            const float a = fabsf(w_nk[c * k + d]);
            if (a > maximum) maximum = a;
        }
        float scale = maximum > 0.0f ? maximum / 127.0f : 1.0f;
        if (scale == 0.0f) scale = 1.0f;
        scales[c] = scale;
        for (int64_t d = 0; d < k; ++d) {
            float r = roundf(w_nk[c * k + d] / scale);
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            q[c * k + d] = (int8_t)r;
        }
    }
}

/* quantized_invoke (next_milestones.cpp:50-69), no bias / relu:
 * y[m,n] = sum_k (x[m,k] * float(q[n,k])) * s_n, sequential over k, fp32
 * activations.  The reference's `acc += x * float(q - zp) * scale` multiplies
 * left to right and, compiled with FMA contraction, adds the scaled product
 * into the accumulator with one fused step: acc = fma(x * q, s, acc).  That
 * is what each output does here; q is laid out [K][N] as exact floats so the
 * chain vectorises across n. */
/* Blocked as sfgo_matmul (same tiles, same per-output chain): the 4 x 32
 * kernel rounds x * q with _mm256_mul_ps and adds it scaled with one fused
 * step, lane by lane what the plain loop does.  Each tile widens its q block
 * (exactly) into panels of 32 output channels, [k block][32], read
 * contiguously; the int8 matrix itself is read once per tile row. */
static void qmm_kernel_4x32(const float* x, int64_t ldx, const float* qp, const float* s,
                            float* c, int64_t ldc, int64_t kn, int first) {
    __m256 acc[4][4];
    const __m256 s0 = _mm256_loadu_ps(s), s1 = _mm256_loadu_ps(s + 8);
    const __m256 s2 = _mm256_loadu_ps(s + 16), s3 = _mm256_loadu_ps(s + 24);
    for (int r = 0; r < 4; ++r)
        for (int v = 0; v < 4; ++v)
            acc[r][v] = first ? _mm256_setzero_ps() : _mm256_loadu_ps(c + r * ldc + 8 * v);
    for (int64_t t = 0; t < kn; ++t) {
        const float* qr = qp + t * 32;
        const __m256 q0 = _mm256_loadu_ps(qr), q1 = _mm256_loadu_ps(qr + 8);
        const __m256 q2 = _mm256_loadu_ps(qr + 16), q3 = _mm256_loadu_ps(qr + 24);
        for (int r = 0; r < 4; ++r) {
            const __m256 xr = _mm256_broadcast_ss(x + r * ldx + t);
            acc[r][0] = _mm256_fmadd_ps(_mm256_mul_ps(xr, q0), s0, acc[r][0]);
            acc[r][1] = _mm256_fmadd_ps(_mm256_mul_ps(xr, q1), s1, acc[r][1]);
            acc[r][2] = _mm256_fmadd_ps(_mm256_mul_ps(xr, q2), s2, acc[r][2]);
            acc[r][3] = _mm256_fmadd_ps(_mm256_mul_ps(xr, q3), s3, acc[r][3]);
        }
    }
    for (int r = 0; r < 4; ++r)
        for (int v = 0; v < 4; ++v) _mm256_storeu_ps(c + r * ldc + 8 * v, acc[r][v]);
}

/* The plain chain, q read as float(q[n][k]) straight from the int8 matrix. */
static void qmm_edge(const float* x, const int8_t* q_nk, const float* scales, float* out,
                     int64_t n, int64_t k, int64_t i0, int64_t i1, int64_t j0, int64_t j1,
                     int64_t k0, int64_t k1) {
    for (int64_t i = i0; i < i1; ++i) {
        float* crow = out + i * n;
        if (k0 == 0)
            for (int64_t j = j0; j < j1; ++j) crow[j] = 0.0f;
        for (int64_t kk = k0; kk < k1; ++kk) {
            const float xik = x[i * k + kk];
            for (int64_t j = j0; j < j1; ++j)
                crow[j] = fmaf(xik * (float)q_nk[j * k + kk], scales[j], crow[j]);
        }
    }
}

void sfgo_quantized_matmul(const float* x, const int8_t* q_nk, const float* scales,
                           int64_t m, int64_t n, int64_t k, float* out) {
    if (k <= 0) {
        for (int64_t i = 0; i < m * n; ++i) out[i] = 0.0f;
        return;
    }
    const int64_t tiles_m = (m + MM_TM - 1) / MM_TM, tiles_n = (n + MM_TN - 1) / MM_TN;
#pragma omp parallel
    {
        /* this thread's widened copy of one q block: MM_TN / 32 panels [MM_TK][32] */
        float* qp = (float*)malloc(sizeof(float) * MM_TK * MM_TN);
#pragma omp for schedule(dynamic, 1)
        for (int64_t t = 0; t < tiles_m * tiles_n; ++t) {
            const int64_t i0 = (t % tiles_m) * MM_TM, j0 = (t / tiles_m) * MM_TN;
            const int64_t i1 = i0 + MM_TM < m ? i0 + MM_TM : m;
            const int64_t j1 = j0 + MM_TN < n ? j0 + MM_TN : n;
            const int64_t i4 = i0 + (i1 - i0) / 4 * 4, j32 = j0 + (j1 - j0) / 32 * 32;
            for (int64_t k0 = 0; k0 < k; k0 += MM_TK) {
                const int64_t k1 = k0 + MM_TK < k ? k0 + MM_TK : k, kn = k1 - k0;
                if (i4 > i0)
                    for (int64_t j = j0; j < j32; j += 32) {
                        float* panel = qp + (j - j0) * MM_TK;
                        for (int c = 0; c < 32; ++c) {
                            const int8_t* row = q_nk + (j + c) * k + k0;
                            for (int64_t kk = 0; kk < kn; ++kk) panel[kk * 32 + c] = (float)row[kk];
                        }
                        for (int64_t i = i0; i < i4; i += 4)
                            qmm_kernel_4x32(x + i * k + k0, k, panel, scales + j, out + i * n + j, n, kn,
                                            k0 == 0);
                    }
                if (j32 < j1) qmm_edge(x, q_nk, scales, out, n, k, i0, i4, j32, j1, k0, k1);
                if (i4 < i1) qmm_edge(x, q_nk, scales, out, n, k, i4, i1, j0, j1, k0, k1);
            }
        }
        free(qp);
    }
}

/* execute_quantized_moe_once (next_milestones.cpp:418-460): per token and slot,
 * gate = x W1q, up = silu(x W3q), out += w * ((gate*up) W2q).  Expert weights
 * are [E][N][K] int8 with per-channel scales [E][N]. */
void sfgo_quantized_moe(const float* x, const int8_t* w1q, const float* s1,
                        const int8_t* w3q, const float* s3, const int8_t* w2q,
                        const float* s2, int64_t tokens, int64_t hidden, int64_t inter,
                        int64_t top_k, const int32_t* ids, const float* weights, float* out) {
    for (int64_t i = 0; i < tokens * hidden; ++i) out[i] = 0.0f;
    int32_t experts = 0;
    for (int64_t i = 0; i < tokens * top_k; ++i)
        if (ids[i] + 1 > experts) experts = ids[i] + 1;
    float* y_all = (float*)calloc((size_t)(tokens * top_k * hidden), sizeof(float));
    for (int32_t e = 0; e < experts; ++e) {
        int64_t rows = 0;
        for (int64_t i = 0; i < tokens * top_k; ++i) rows += ids[i] == e;
        if (rows == 0) continue;
        float* xe = (float*)malloc(sizeof(float) * (size_t)(rows * hidden));
        int64_t* where = (int64_t*)malloc(sizeof(int64_t) * (size_t)rows);
        int64_t r = 0;
        for (int64_t i = 0; i < tokens * top_k; ++i)
            if (ids[i] == e) {
                where[r] = i;
                memcpy(xe + r * hidden, x + (i / top_k) * hidden, sizeof(float) * (size_t)hidden);
                ++r;
            }
        float* gate = (float*)malloc(sizeof(float) * (size_t)(rows * inter));
        float* up = (float*)malloc(sizeof(float) * (size_t)(rows * inter));
        float* y = (float*)malloc(sizeof(float) * (size_t)(rows * hidden));
        sfgo_quantized_matmul(xe, w1q + (int64_t)e * inter * hidden, s1 + (int64_t)e * inter,
                              rows, inter, hidden, gate);
        sfgo_quantized_matmul(xe, w3q + (int64_t)e * inter * hidden, s3 + (int64_t)e * inter,
                              rows, inter, hidden, up);
        for (int64_t i = 0; i < rows * inter; ++i) {
            const float u = up[i] / (1.0f + expf(-up[i]));
            gate[i] = gate[i] * u;
        }
        sfgo_quantized_matmul(gate, w2q + (int64_t)e * hidden * inter, s2 + (int64_t)e * hidden,
                              rows, hidden, inter, y);
        for (int64_t i = 0; i < rows; ++i)
            memcpy(y_all + where[i] * hidden, y + i * hidden, sizeof(float) * (size_t)hidden);
        free(xe); free(where); free(gate); free(up); free(y);
    }
    for (int64_t t = 0; t < tokens; ++t)
        for (int64_t s = 0; s < top_k; ++s) {
            const float w = weights[t * top_k + s];
            const float* y = y_all + (t * top_k + s) * hidden;
            for (int64_t f = 0; f < hidden; ++f)
                out[t * hidden + f] = fmaf(w, y[f], out[t * hidden + f]);
        }
    free(y_all);
}

/* max_abs_error (runtime.cpp:628-635): |float(a - b)| in double, folded with
 * std::max(error, d) = (error < d ? d : error), so a NaN difference leaves the
 * running value unchanged. */
double sfgo_max_abs_error(const float* a, const float* b, int64_t count) {
    double err = 0.0;
    for (int64_t i = 0; i < count; ++i) {
        const double d = fabs((double)(a[i] - b[i]));
        err = err < d ? d : err;
    }
    return err;
}

/* ------------------------------------------------------------------------- */
/* Whole layer: reference_decoder_layer (decoder_compiler.cpp:622-673); int8  */
/* mode follows execute_quantized_decoder_once (next_milestones.cpp:339-385)  */
/* for the projections and execute_quantized_moe_once (418-460) for experts.  */
/* Decode (context > 0) attends only over the cached K/V and applies RoPE at  */
/* the position within the new tokens (decoder_compiler.cpp:238-243, 640-645).*/
/* ------------------------------------------------------------------------- */

static float* alloc_f(int64_t n) { return (float*)calloc((size_t)n, sizeof(float)); }

int sfgo_decoder_layer(const sfgo_layer_cfg* c, const sfgo_layer_data* d, float* out,
                       sfgo_layer_taps* taps) {
#ifdef _OPENMP
    if (c->threads > 0) omp_set_num_threads(c->threads);
#endif
    if (c->batch <= 0 || c->sequence <= 0 || c->hidden <= 0 || c->intermediate <= 0 ||
        c->query_heads <= 0 || c->kv_heads <= 0 || c->head_dim <= 0 ||
        c->hidden != c->query_heads * c->head_dim || c->query_heads % c->kv_heads != 0 ||
        c->rms_epsilon <= 0.0f)
        return 1;
    if (c->moe && (c->experts <= 0 || c->top_k <= 0 || c->top_k > c->experts)) return 1;
    const int64_t rows = (int64_t)c->batch * c->sequence;
    const int64_t H = c->hidden, I = c->intermediate, D = c->head_dim;
    const int64_t kvd = (int64_t)c->kv_heads * D;
    const int64_t qkvw = H + 2 * kvd;

    float* n1 = alloc_f(rows * H);
    sfgo_rms_norm(d->input, d->rms1, n1, rows, H, c->rms_epsilon);
    float* qkv = alloc_f(rows * qkvw);
    if (c->int8_weights) {
        float* part = alloc_f(rows * H);
        sfgo_quantized_matmul(n1, d->q8[0], d->s8[0], rows, H, H, part);
        for (int64_t r = 0; r < rows; ++r) memcpy(qkv + r * qkvw, part + r * H, sizeof(float) * (size_t)H);
        sfgo_quantized_matmul(n1, d->q8[1], d->s8[1], rows, kvd, H, part);
        for (int64_t r = 0; r < rows; ++r) memcpy(qkv + r * qkvw + H, part + r * kvd, sizeof(float) * (size_t)kvd);
        sfgo_quantized_matmul(n1, d->q8[2], d->s8[2], rows, kvd, H, part);
        for (int64_t r = 0; r < rows; ++r) memcpy(qkv + r * qkvw + H + kvd, part + r * kvd, sizeof(float) * (size_t)kvd);
        free(part);
    } else {
        float* packed = alloc_f(H * qkvw);
        const float* ws[3] = {d->wq, d->wk, d->wv};
        const int64_t widths[3] = {H, kvd, kvd};
        sfgo_concat_columns(ws, widths, 3, H, packed);
        sfgo_matmul(n1, packed, qkv, rows, qkvw, H);
        free(packed);
    }
    const int64_t qn = rows * H, kn = rows * kvd;
    float* q = alloc_f(qn);
    float* k = alloc_f(kn);
    float* v = alloc_f(kn);
    const int append = c->context > 0 && c->kv_append;
    if (append) {
        /* Append mode (the build's non-reference option): the step's tokens are
         * rotated at their true positions context + s, stored in the pool dtype
         * (bf16, or fp32 on the fp32 path) after the cached tokens, and
         * attended over with the cache. */
        sfgo_split_qkv_rope(qkv, c->batch, c->sequence, H, c->query_heads, c->kv_heads, D,
                            c->rope_theta, q, k, v);
        /* Q and K again from the unrotated rows, rotated at the new positions */
        for (int64_t b = 0; b < c->batch; ++b)
            for (int64_t s = 0; s < c->sequence; ++s) {
                const float* row = qkv + (b * c->sequence + s) * qkvw;
                for (int64_t h = 0; h < c->query_heads; ++h)
                    memcpy(q + ((b * c->query_heads + h) * c->sequence + s) * D, row + h * D,
                           sizeof(float) * (size_t)D);
                for (int64_t h = 0; h < c->kv_heads; ++h)
                    memcpy(k + ((b * c->kv_heads + h) * c->sequence + s) * D, row + H + h * D,
                           sizeof(float) * (size_t)D);
            }
        sfgo_rope_at(q, c->batch, c->query_heads, c->sequence, D, c->rope_theta, c->context);
        sfgo_rope_at(k, c->batch, c->kv_heads, c->sequence, D, c->rope_theta, c->context);
        if (!c->kv_pool_f32) {
            sfgo_round_bf16(k, kn);
            sfgo_round_bf16(v, kn);
        }
    } else {
        sfgo_split_qkv_rope(qkv, c->batch, c->sequence, H, c->query_heads, c->kv_heads, D,
                            c->rope_theta, q, k, v);
    }
    const int64_t skv = c->context > 0 ? c->context + (append ? c->sequence : 0) : c->sequence;
    sfgo_attn_cfg ac = {c->batch, c->query_heads, c->kv_heads, c->sequence, skv, c->head_dim,
                        c->head_dim, c->causal, 0.0f};
    float* attn = alloc_f(qn);
    if (append) {
        float* kc = alloc_f((int64_t)c->batch * c->kv_heads * skv * D);
        float* vc = alloc_f((int64_t)c->batch * c->kv_heads * skv * D);
        for (int64_t b = 0; b < c->batch; ++b)
            for (int64_t h = 0; h < c->kv_heads; ++h) {
                const int64_t bh = b * c->kv_heads + h;
                memcpy(kc + bh * skv * D, d->cached_k + bh * c->context * D, sizeof(float) * (size_t)(c->context * D));
                memcpy(vc + bh * skv * D, d->cached_v + bh * c->context * D, sizeof(float) * (size_t)(c->context * D));
                memcpy(kc + (bh * skv + c->context) * D, k + bh * c->sequence * D, sizeof(float) * (size_t)(c->sequence * D));
                memcpy(vc + (bh * skv + c->context) * D, v + bh * c->sequence * D, sizeof(float) * (size_t)(c->sequence * D));
            }
        sfgo_attention(&ac, q, kc, vc, attn);
        if (taps && taps->new_k) memcpy(taps->new_k, k, sizeof(float) * (size_t)kn);
        if (taps && taps->new_v) memcpy(taps->new_v, v, sizeof(float) * (size_t)kn);
        free(kc); free(vc);
    } else if (c->context > 0) {
        sfgo_attention(&ac, q, d->cached_k, d->cached_v, attn);
    } else {
        sfgo_attention(&ac, q, k, v, attn);
    }
    float* merged = alloc_f(rows * H);
    sfgo_merge_heads(attn, c->batch, c->sequence, c->query_heads, D, merged);
    float* proj = alloc_f(rows * H);
    if (c->int8_weights)
        sfgo_quantized_matmul(merged, d->q8[3], d->s8[3], rows, H, H, proj);
    else
        sfgo_matmul(merged, d->wo, proj, rows, H, H);
    float* r1 = alloc_f(rows * H);
    sfgo_add(proj, d->input, r1, rows * H);
    float* n2 = alloc_f(rows * H);
    sfgo_rms_norm(r1, d->rms2, n2, rows, H, c->rms_epsilon);
    float* ffn = alloc_f(rows * H);
    if (!c->moe) {
        float* act = alloc_f(rows * I);
        if (c->int8_weights) {
            float* g = alloc_f(rows * I);
            float* u = alloc_f(rows * I);
            sfgo_quantized_matmul(n2, d->q8[4], d->s8[4], rows, I, H, g);
            sfgo_quantized_matmul(n2, d->q8[5], d->s8[5], rows, I, H, u);
            for (int64_t i = 0; i < rows * I; ++i) act[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
            sfgo_quantized_matmul(act, d->q8[6], d->s8[6], rows, H, I, ffn);
            free(g); free(u);
        } else {
            float* packed = alloc_f(H * 2 * I);
            const float* ws[2] = {d->wg, d->wu};
            const int64_t widths[2] = {I, I};
            sfgo_concat_columns(ws, widths, 2, H, packed);
            float* gu = alloc_f(rows * 2 * I);
            sfgo_matmul(n2, packed, gu, rows, 2 * I, H);
            sfgo_swiglu(gu, rows, I, act);
            sfgo_matmul(act, d->wd, ffn, rows, H, I);
            free(packed); free(gu);
        }
        free(act);
    } else {
        int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows * c->top_k));
        float* wts = alloc_f(rows * c->top_k);
        int32_t* counts = (int32_t*)calloc((size_t)c->experts, sizeof(int32_t));
        if (d->trace_ids) {
            memcpy(ids, d->trace_ids, sizeof(int32_t) * (size_t)(rows * c->top_k));
            memcpy(wts, d->trace_weights, sizeof(float) * (size_t)(rows * c->top_k));
            for (int64_t i = 0; i < rows * c->top_k; ++i) counts[ids[i]] += 1;
        } else {
            sfgo_route_topk(n2, d->router, d->router_bias, rows, H, c->experts, c->top_k, ids,
                            wts, counts);
        }
        if (c->int8_weights)
            sfgo_quantized_moe(n2, d->e1q, d->e1s, d->e3q, d->e3s, d->e2q, d->e2s, rows, H, I,
                               c->top_k, ids, wts, ffn);
        else
            sfgo_moe_reference(n2, d->w1, d->w3, d->w2, rows, H, I, c->top_k, ids, wts, ffn);
        if (taps && taps->ids) memcpy(taps->ids, ids, sizeof(int32_t) * (size_t)(rows * c->top_k));
        if (taps && taps->weights) memcpy(taps->weights, wts, sizeof(float) * (size_t)(rows * c->top_k));
        if (taps && taps->counts) memcpy(taps->counts, counts, sizeof(int32_t) * (size_t)c->experts);
        free(ids); free(wts); free(counts);
    }
    sfgo_add(r1, ffn, out, rows * H);
    if (taps) {
        if (taps->normalized1) memcpy(taps->normalized1, n1, sizeof(float) * (size_t)(rows * H));
        if (taps->qkv) memcpy(taps->qkv, qkv, sizeof(float) * (size_t)(rows * qkvw));
        if (taps->attn_merged) memcpy(taps->attn_merged, merged, sizeof(float) * (size_t)(rows * H));
        if (taps->residual1) memcpy(taps->residual1, r1, sizeof(float) * (size_t)(rows * H));
        if (taps->normalized2) memcpy(taps->normalized2, n2, sizeof(float) * (size_t)(rows * H));
    }
    free(n1); free(qkv); free(q); free(k); free(v); free(attn); free(merged); free(proj);
    free(r1); free(n2); free(ffn);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* The whole layer at a sample of query rows (prefill).  Same arithmetic as   */
/* sfgo_decoder_layer restricted to rows sample[0..n) (row = b * S + s):      */
/* RMSNorm and the K / V projections run for every row (a query attends over  */
/* every earlier key), Q, attention, O-projection, residual, RMSNorm and FFN  */
/* only for the sampled rows.  Each output element is the same chain as in    */
/* the full layer (products are per-column FMA chains over k; attention and   */
/* the FFN are per row), so every sampled row of `out` and of the taps (n     */
/* rows each) equals that row of sfgo_decoder_layer bit for bit.              */
/* ------------------------------------------------------------------------- */

static void gather_rows(const float* src, const int64_t* sample, int64_t n, int64_t width,
                        float* dst) {
    for (int64_t i = 0; i < n; ++i)
        memcpy(dst + i * width, src + sample[i] * width, sizeof(float) * (size_t)width);
}

int sfgo_decoder_layer_rows(const sfgo_layer_cfg* c, const sfgo_layer_data* d,
                            const int64_t* sample, int64_t n, float* out,
                            sfgo_layer_taps* taps) {
#ifdef _OPENMP
    if (c->threads > 0) omp_set_num_threads(c->threads);
#endif
    if (c->batch <= 0 || c->sequence <= 0 || c->hidden <= 0 || c->intermediate <= 0 ||
        c->query_heads <= 0 || c->kv_heads <= 0 || c->head_dim <= 0 ||
        c->hidden != c->query_heads * c->head_dim || c->query_heads % c->kv_heads != 0 ||
        c->rms_epsilon <= 0.0f || c->context != 0 || c->kv_append || n <= 0)
        return 1;
    if (c->moe && (c->experts <= 0 || c->top_k <= 0 || c->top_k > c->experts)) return 1;
    const int64_t B = c->batch, S = c->sequence;
    const int64_t rows = B * S;
    for (int64_t i = 0; i < n; ++i)
        if (sample[i] < 0 || sample[i] >= rows) return 1;
    const int64_t H = c->hidden, I = c->intermediate, D = c->head_dim;
    const int64_t Hq = c->query_heads, Hkv = c->kv_heads;
    const int64_t kvd = Hkv * D;

    /* every row: normalised input, K and V (RoPE on K at the index within S) */
    float* n1 = alloc_f(rows * H);
    sfgo_rms_norm(d->input, d->rms1, n1, rows, H, c->rms_epsilon);
    float* kvp = alloc_f(rows * 2 * kvd);
    if (c->int8_weights) {
        float* part = alloc_f(rows * kvd);
        for (int j = 0; j < 2; ++j) {
            sfgo_quantized_matmul(n1, d->q8[1 + j], d->s8[1 + j], rows, kvd, H, part);
            for (int64_t r = 0; r < rows; ++r)
                memcpy(kvp + r * 2 * kvd + j * kvd, part + r * kvd, sizeof(float) * (size_t)kvd);
        }
        free(part);
    } else {
        float* packed = alloc_f(H * 2 * kvd);
        const float* ws[2] = {d->wk, d->wv};
        const int64_t widths[2] = {kvd, kvd};
        sfgo_concat_columns(ws, widths, 2, H, packed);
        sfgo_matmul(n1, packed, kvp, rows, 2 * kvd, H);
        free(packed);
    }
    float* k = alloc_f(rows * kvd);
    float* v = alloc_f(rows * kvd);
    for (int64_t b = 0; b < B; ++b)
        for (int64_t s = 0; s < S; ++s)
            for (int64_t h = 0; h < Hkv; ++h) {
                const float* row = kvp + (b * S + s) * 2 * kvd;
                memcpy(k + ((b * Hkv + h) * S + s) * D, row + h * D, sizeof(float) * (size_t)D);
                memcpy(v + ((b * Hkv + h) * S + s) * D, row + kvd + h * D, sizeof(float) * (size_t)D);
            }
    sfgo_rope(k, B, Hkv, S, D, c->rope_theta);

    /* sampled rows: Q (RoPE at the row's index within S) and attention */
    float* n1s = alloc_f(n * H);
    gather_rows(n1, sample, n, H, n1s);
    float* qs = alloc_f(n * H);
    if (c->int8_weights)
        sfgo_quantized_matmul(n1s, d->q8[0], d->s8[0], n, H, H, qs);
    else
        sfgo_matmul(n1s, d->wq, qs, n, H, H);
    float* qrot = alloc_f(n * H);
    memcpy(qrot, qs, sizeof(float) * (size_t)(n * H));
    for (int64_t i = 0; i < n; ++i)  /* row i holds [Hq][D] of one token */
        sfgo_rope_at(qrot + i * H, 1, Hq, 1, D, c->rope_theta, sample[i] % S);
    sfgo_attn_cfg ac = {c->batch, c->query_heads, c->kv_heads, c->sequence, c->sequence,
                        c->head_dim, c->head_dim, c->causal, 0.0f};
    const float scale = attention_scale(&ac);
    float* merged = alloc_f(n * H);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t ih = 0; ih < n * Hq; ++ih) {
        const int64_t i = ih / Hq, h = ih % Hq;
        const int64_t b = sample[i] / S, s = sample[i] % S;
        const int64_t kvh = h * Hkv / Hq;
        float* scores = (float*)malloc(sizeof(float) * (size_t)S);
        attention_row(qrot + i * H + h * D, k + (b * Hkv + kvh) * S * D, v + (b * Hkv + kvh) * S * D,
                      S, c->causal ? s : S - 1, D, D, scale, scores, merged + i * H + h * D);
        free(scores);
    }
    /* O-projection, residual, RMSNorm, FFN on the sampled rows */
    float* proj = alloc_f(n * H);
    if (c->int8_weights)
        sfgo_quantized_matmul(merged, d->q8[3], d->s8[3], n, H, H, proj);
    else
        sfgo_matmul(merged, d->wo, proj, n, H, H);
    float* xs = alloc_f(n * H);
    gather_rows(d->input, sample, n, H, xs);
    float* r1 = alloc_f(n * H);
    sfgo_add(proj, xs, r1, n * H);
    float* n2 = alloc_f(n * H);
    sfgo_rms_norm(r1, d->rms2, n2, n, H, c->rms_epsilon);
    float* ffn = alloc_f(n * H);
    if (!c->moe) {
        float* act = alloc_f(n * I);
        if (c->int8_weights) {
            float* g = alloc_f(n * I);
            float* u = alloc_f(n * I);
            sfgo_quantized_matmul(n2, d->q8[4], d->s8[4], n, I, H, g);
            sfgo_quantized_matmul(n2, d->q8[5], d->s8[5], n, I, H, u);
            for (int64_t i = 0; i < n * I; ++i) act[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
            sfgo_quantized_matmul(act, d->q8[6], d->s8[6], n, H, I, ffn);
            free(g); free(u);
        } else {
            float* packed = alloc_f(H * 2 * I);
            const float* ws[2] = {d->wg, d->wu};
            const int64_t widths[2] = {I, I};
            sfgo_concat_columns(ws, widths, 2, H, packed);
            float* gu = alloc_f(n * 2 * I);
            sfgo_matmul(n2, packed, gu, n, 2 * I, H);
            sfgo_swiglu(gu, n, I, act);
            sfgo_matmul(act, d->wd, ffn, n, H, I);
            free(packed); free(gu);
        }
        free(act);
    } else {
        const int64_t K = c->top_k;
        int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n * K));
        float* wts = alloc_f(n * K);
        int32_t* counts = (int32_t*)calloc((size_t)c->experts, sizeof(int32_t));
        if (d->trace_ids) {
            for (int64_t i = 0; i < n; ++i)
                for (int64_t j = 0; j < K; ++j) {
                    ids[i * K + j] = d->trace_ids[sample[i] * K + j];
                    wts[i * K + j] = d->trace_weights[sample[i] * K + j];
                    counts[ids[i * K + j]] += 1;
                }
        } else {
            sfgo_route_topk(n2, d->router, d->router_bias, n, H, c->experts, K, ids, wts, counts);
        }
        if (c->int8_weights)
            sfgo_quantized_moe(n2, d->e1q, d->e1s, d->e3q, d->e3s, d->e2q, d->e2s, n, H, I, K, ids,
                               wts, ffn);
        else
            sfgo_moe_reference(n2, d->w1, d->w3, d->w2, n, H, I, K, ids, wts, ffn);
        if (taps && taps->ids) memcpy(taps->ids, ids, sizeof(int32_t) * (size_t)(n * K));
        if (taps && taps->weights) memcpy(taps->weights, wts, sizeof(float) * (size_t)(n * K));
        if (taps && taps->counts) memcpy(taps->counts, counts, sizeof(int32_t) * (size_t)c->experts);
        free(ids); free(wts); free(counts);
    }
    sfgo_add(r1, ffn, out, n * H);
    if (taps) {
        if (taps->normalized1) memcpy(taps->normalized1, n1s, sizeof(float) * (size_t)(n * H));
        if (taps->qkv)
            for (int64_t i = 0; i < n; ++i) {
                float* row = taps->qkv + i * (H + 2 * kvd);
                memcpy(row, qs + i * H, sizeof(float) * (size_t)H);
                memcpy(row + H, kvp + sample[i] * 2 * kvd, sizeof(float) * (size_t)(2 * kvd));
            }
        if (taps->attn_merged) memcpy(taps->attn_merged, merged, sizeof(float) * (size_t)(n * H));
        if (taps->residual1) memcpy(taps->residual1, r1, sizeof(float) * (size_t)(n * H));
        if (taps->normalized2) memcpy(taps->normalized2, n2, sizeof(float) * (size_t)(n * H));
    }
    free(n1); free(kvp); free(k); free(v); free(n1s); free(qs); free(qrot); free(merged);
    free(proj); free(xs); free(r1); free(n2); free(ffn);
    return 0;
}
