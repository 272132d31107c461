/*
 * sfg_hip.h -- C ABI of the MI355X (gfx950) execution backend for SchedForge's
 * compiled decoder layer.  Library: schedforge_amd/lib/libsfg_hip.so.
 *
 * Conventions (after the reference's only C ABI, `schedforge_matmul_v1`,
 * src/llvm_backend.cpp:39-40, 62-64, and its metadata symbol, 622-643):
 *   - versioned `_v1` names, int64_t sizes, raw device pointers, no C++ types;
 *   - every entry point returns 0 on success, SFG_ERR_* otherwise, and never
 *     throws.  Codes below 16 are configuration / shape / guard violations
 *     (the reference throws std::invalid_argument for these); codes from 16 up
 *     are device or resource failures (the reference's std::runtime_error).
 *     sfg_hip_last_error() returns this thread's message for the last failure;
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream); kernels
 *     are enqueued asynchronously on it.  Calls sharing a stream must be
 *     serialised by the caller; independent calls may run on different streams;
 *   - the library allocates no device memory: callers pass workspaces sized by
 *     the *_workspace_v1 queries.
 *
 * Device layouts (all row-major):
 *   activations   [rows][H] fp32 (residual stream) / bf16 (GEMM operands)
 *   weights       [N][K] -- output channel major, K contiguous.  The reference
 *                 keeps [K][N] fp32 (decoder_compiler.h:34-49) and packs
 *                 Wq|Wk|Wv and Wg|Wu by columns (decoder_compiler.cpp:535-552);
 *                 sfg_hip_pack_weight_v1 produces the transposed packed form.
 *                 int8 weights are [N][K] with per-channel fp32 scales, exactly
 *                 the reference's QuantizedMatMulWeights (next_milestones.h:52-56).
 *   tiled weights SFG_LAYOUT_TILED (decode plans): the [N][K] matrix cut into
 *                 16-row x 128-k tiles stored [N/16][K/128] contiguously, each
 *                 tile in MFMA-fragment order -- bf16: 4 x [64 lanes][8 values]
 *                 with lane l = 16 g + r holding row r, k = 32 s + 8 g + [0,8)
 *                 for fragment s; int8: 2 x [64 lanes][16 values] with k =
 *                 32 g + 16 t + [0,16) -- so every load a wave issues reads 1 KB
 *                 contiguous.  Same bytes as [N][K].
 *   paged KV      K pool [page][Hkv][page_tokens][D], V pool
 *                 [page][Hkv][D][page_tokens] (token-minor inside a page:
 *                 the decode kernel reads V^T operands as 8-byte runs), bf16
 *                 (fp32 on the fp32 path); each (page, kv_head) is one
 *                 contiguous 4 KB run at D=128, 16-token bf16 pages.  One
 *                 page-table row per sequence [B][pages_per_seq].
 */
#ifndef SFG_HIP_H
#define SFG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SFG_HIP_ABI_VERSION 1

enum sfg_status {
    SFG_OK = 0,
    SFG_ERR_INVALID_CONFIG = 1, /* decoder_compiler.cpp:26-39 validate()            */
    SFG_ERR_SHAPE = 2,          /* shape / layout mismatch (attention_compiler.cpp:31-41) */
    SFG_ERR_GUARD = 3,          /* compiled guard violated (context > capacity, page id) */
    SFG_ERR_UNSUPPORTED = 4,    /* configuration valid but not lowered on gfx950  */
    SFG_ERR_ABI = 5,            /* descriptor ABI version mismatch               */
    SFG_ERR_DEVICE = 16,        /* HIP runtime error                             */
    SFG_ERR_WORKSPACE = 17      /* workspace too small                           */
};

enum sfg_dtype { SFG_F32 = 0, SFG_BF16 = 1, SFG_I8 = 2, SFG_I32 = 3 /* taps only */ };

enum sfg_layout { SFG_LAYOUT_NK = 0, SFG_LAYOUT_TILED = 1 };

/* Output tile of the bf16 direct-to-LDS GEMM family that runs the prefill
 * projections and grouped expert GEMMs (bf16 weights, >= 1024 rows, k % 32 == 0).
 * A plan policy, not a numeric choice: every tile gives bit-identical results
 * (each output is one fp32 accumulation in k order).  Ignored by the other GEMM
 * paths (skinny decode GEMV, fp32, int8 and small-M kernels).  The plan
 * optimiser (ExecutablePlanOptimizer, decoder_compiler.cpp:750-861) searches it. */
enum sfg_gemm_tile {
    SFG_TILE_AUTO = 0,       /* the largest tile that still gives >= 512 workgroups
                                (256 x 256 as V); grouped products take V from 128
                                workgroups up                                       */
    SFG_TILE_256x256_PP = 1, /* eight waves as two ping-pong groups of four          */
    SFG_TILE_256x256_W8 = 2, /* eight waves (2 x 4), 128 x 64 per wave               */
    SFG_TILE_256x256_W4 = 3, /* four waves (2 x 2), 128 x 128 per wave               */
    SFG_TILE_256x128 = 4,    /* four waves, two workgroups per CU                    */
    SFG_TILE_128x256 = 5,
    SFG_TILE_128x128 = 6,
    SFG_TILE_256x256_V = 7,  /* four waves (2 x 2), 64-k slabs by LDS DMA, A in two
                                stages and B in three (160 KB of LDS)               */
    SFG_TILE_COUNT = 8
};

enum sfg_epilogue {
    SFG_EPI_NONE = 0,      /* C = A B                                             */
    SFG_EPI_RESIDUAL = 1,  /* C = A B + R  (R fp32 [M][N]); decoder_compiler.cpp:256,277 */
    SFG_EPI_SWIGLU = 2,    /* B is [2N][K]: rows [0,N) gate, [N,2N) up;
                              C = silu(A Bg) * (A Bu); decoder_compiler.cpp:183-194 */
    SFG_EPI_GLU_SILU_UP = 3 /* MoE form: C = (A B1) * silu(A B3), B = [W1 ; W3];
                              moe_compiler.cpp:143-149                          */
};

/* ---------------- library identity ---------------- */
int sfg_hip_abi_version(void);
/* key=value;... invariants of this build (after schedforge_aot_metadata_v1,
 * llvm_backend.cpp:622-643): abi, arch, dtypes, the activation dtypes and the
 * weight dtypes each takes, layouts, the lowered envelope (head_dim 1..256,
 * any page size, any new-token count per decode step, dense and MoE FFNs) and
 * the shapes the MFMA kernels take (mfma_decode, mfma_prefill, mfma_gemm);
 * the other shapes run the row-per-wave attention and VALU GEMM kernels. */
const char* sfg_hip_metadata_v1(void);
const char* sfg_hip_last_error(void);
/* CUs, XCDs (hipDeviceAttributeNumberOfXccs) and HBM bytes of a device. */
int sfg_hip_device_info_v1(int device, int* cu_count, int* xcd_count, int64_t* hbm_bytes);

/* The GPU target a plan compiles for: the counterpart of the reference's
 * TargetInfo (include/schedforge/schedforge.h:15-34, TargetInfo::detect in
 * src/target.cpp:8-17), which describes the CPU the LoopIR schedules target.
 * Queried from the device (architecture, CUs, XCDs, LDS, L2, clocks, HBM);
 * peaks follow from the queried counts and clock with gfx950's per-CU rates
 * (bf16 dense MFMA 4096 FLOP / clock / CU, fp32 VALU 256 FLOP / clock / CU);
 * HBM bandwidth is gfx950's published 8 TB/s (HIP's memory clock and bus
 * width understate HBM3E's data rate), else estimated from them. */
typedef struct {
    char architecture[64];        /* gcnArchName, e.g. gfx950:sramecc+:xnack- */
    int32_t wavefront;            /* 64 */
    int32_t compute_units;        /* 256 on MI355X */
    int32_t xcds;                 /* accelerator complex dies, workgroups dealt round-robin */
    int32_t simds_per_cu;         /* 4 */
    int64_t lds_bytes_per_cu;     /* 160 KiB on gfx950 */
    int64_t l2_bytes_per_xcd;     /* 4 MiB on gfx950 */
    int64_t hbm_bytes;            /* device memory */
    double engine_clock_ghz;      /* max engine clock */
    double hbm_gbps;              /* peak HBM bandwidth, GB/s */
    double mfma_bf16_tflops;      /* dense bf16 MFMA peak at engine_clock_ghz */
    double valu_fp32_tflops;      /* fp32 VALU peak (no packed math) */
} sfg_target_info;
int sfg_hip_target_info_v1(int device, sfg_target_info* info);

/* ---------------- constant packing (DecoderCompiler::compile constant
 * specialisation, decoder_compiler.cpp:535-552; quantize_matmul_weights,
 * next_milestones.cpp:611-637) ---------------- */

/* src fp32 [K][N] (ld_src >= N) -> dst [N][K] in dtype (SFG_F32 or SFG_BF16),
 * layout SFG_LAYOUT_NK or SFG_LAYOUT_TILED (bf16, N % 16 == 0, K % 128 == 0). */
int sfg_hip_pack_weight_v1(const float* src, int64_t k, int64_t n, int64_t ld_src, void* dst,
                           int dst_dtype, int layout, void* stream);
/* src fp32 [K][N] -> int8 [N][K] (layout NK or TILED) + scales[N]:
 * s = max|w|/127 (1 if zero), q = clamp(round-half-away(w/s), -127, 127). */
int sfg_hip_quantize_weight_v1(const float* src, int64_t k, int64_t n, int8_t* dst,
                               float* scales, int layout, void* stream);
/* Weight layout the GEMM family reads fastest for a product with `rows`
 * activation rows (grouped: total dispatched rows) and reduction length k. */
int sfg_hip_preferred_weight_layout_v1(int64_t rows, int64_t k, int grouped);
/* fp32 -> bf16 bits, round to nearest even (compiler.cpp:34-43). */
int sfg_hip_to_bf16_v1(const float* src, uint16_t* dst, int64_t count, void* stream);
/* RoPE table [seq][head_dim/2][2] = (cos, sin) of float(pos) * powf(theta, -(2i)/D),
 * computed on the HOST with the reference's float expressions
 * (decoder_compiler.cpp:101-106).  Plain host memory.  An odd head_dim has
 * (head_dim - 1) / 2 pairs; its last dimension is never rotated. */
int sfg_hip_rope_table_host_v1(float* table, int64_t seq, int64_t head_dim, float theta);

/* ---------------- per-op kernels ---------------- */

/* rms_norm (decoder_compiler.cpp:41-62): y = x * (1/sqrtf(float(sum x^2 / H) + eps)) * w,
 * sum in double.  x fp32 [rows][width]; y fp32 or bf16. */
int sfg_hip_rmsnorm_v1(const float* x, const float* w, void* y, int y_dtype, int64_t rows,
                       int64_t width, float eps, void* stream);

/* C[M][N] = A[M][K] * B^T with B stored [N][K] (or [2N][K] for GLU epilogues).
 * a_dtype: SFG_F32 (only with b_dtype SFG_F32) or SFG_BF16.  b_dtype: SFG_F32,
 * SFG_BF16 or SFG_I8 (then b_scales[N or 2N] per output channel).
 * bf16 / int8 operands: a and b 16-byte aligned, lda * 2 and ldb * (2 or 1)
 * bytes multiples of 16 (rows are read as 16-byte vectors), else
 * SFG_ERR_UNSUPPORTED.
 * c_dtype: SFG_F32 or SFG_BF16.  Replaces execute(LoopIR) (runtime.cpp:581-626)
 * for the four projections and quantized_invoke (next_milestones.cpp:50-69).
 * workspace: sfg_hip_gemm_workspace_v1 bytes.  Non-zero only for 33..64 dense
 * rows with k a multiple of 512 (>= 1024) and N (2N for GLU) a multiple of
 * 128: those run split-K over 512-k slices with fp32 partial sums in the
 * workspace, summed in slice order.  With a smaller workspace (or NULL) the
 * same shapes run the single-pass decode kernel instead.
 * b_layout SFG_LAYOUT_TILED is read by the decode GEMV only: bf16 / int8 B,
 * at most 64 rows (grouped: 512 in all), K % 128 == 0 and N % 16 == 0;
 * other shapes with tiled B return SFG_ERR_UNSUPPORTED. */
typedef struct {
    const void* a; int32_t a_dtype; int64_t lda;
    const void* b; int32_t b_dtype; int64_t ldb; const float* b_scales;
    void* c; int32_t c_dtype; int64_t ldc;
    const float* residual; int64_t ldr;
    int64_t m, n, k;
    int32_t epilogue;
    int32_t b_layout;   /* SFG_LAYOUT_NK or SFG_LAYOUT_TILED */
    int32_t tile;       /* sfg_gemm_tile; SFG_TILE_AUTO (0) picks per shape */
} sfg_gemm_args;
size_t sfg_hip_gemm_workspace_v1(int64_t m, int64_t n, int64_t k);
int sfg_hip_gemm_v1(const sfg_gemm_args* args, void* workspace, size_t workspace_bytes,
                    void* stream);
/* The grouped product of execute_moe's expert tasks (compute_task +
 * execute_loop_kernel, moe_compiler.cpp:64-155) in general form: arguments as
 * sfg_hip_gemm_v1 with m the total rows; group g computes output rows
 * [offsets[g], offsets[g + 1]) (device int32, groups + 1 entries, clamped to
 * [0, m]) from A rows a_rows[r] (device int32; NULL: row r; ids outside
 * [0, a_rows_limit) read as zero rows) with the B matrix and scales of group g
 * at b + g * b_group_stride elements and b_scales + g * s_group_stride.
 * Epilogue none, SwiGLU or the MoE GLU (no residual). */
int sfg_hip_gemm_grouped_v1(const sfg_gemm_args* args, const int32_t* a_rows, int64_t a_rows_limit,
                            const int32_t* offsets, int groups, int64_t b_group_stride,
                            int64_t s_group_stride, void* workspace, size_t workspace_bytes,
                            void* stream);

/* split_qkv + apply_rope (decoder_compiler.cpp:96-148).  qkv fp32
 * [B*S][H + 2 Hkv D]; rope_table [S][D/2][2] device copy of
 * sfg_hip_rope_table_host_v1.  q [B][Hq][S][D], k/v [B][Hkv][S][D] in out_dtype
 * (k and v may be NULL: a decode step discards them, decoder_compiler.cpp:238-243).
 * Any head_dim: an odd one's last dimension is copied unrotated (apply_rope's
 * pair loop stops at d + 1 < D); rope_table may be NULL when head_dim is 1. */
int sfg_hip_qkv_split_rope_v1(const float* qkv, const float* rope_table, int64_t batch,
                              int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                              void* q, void* k, void* v, int out_dtype, void* stream);

/* IO-aware causal/non-causal GQA prefill, online softmax
 * (attention_compiler.cpp:286-377).  q [B][Hq][Sq][D], k/v [B][Hkv][Skv][D] in dtype
 * (SFG_F32 or SFG_BF16); out is written merged [B*Sq][Hq*D] in out_dtype
 * (merge_attention, decoder_compiler.cpp:150-174).  scale <= 0: 1/sqrt(D). */
int sfg_hip_attn_prefill_v1(const void* q, const void* k, const void* v, void* out,
                            int dtype, int out_dtype, int64_t batch, int64_t q_heads,
                            int64_t kv_heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                            int causal, float scale, void* stream);

/* The same prefill (attention_compiler.cpp:286-377) over a transposed value
 * tensor -- the layout the gfx950 flash kernel streams: q [B][Hq][Sq][128],
 * k [B][Hkv][Skv][128], vt [B][Hkv][128][ld_vt] bf16 with
 * ld_vt = sfg_hip_attn_vt_ld_v1(Skv) and keys in [Skv, ld_vt) zero.  head_dim
 * must be 128.  sfg_hip_qkv_split_rope_vt_v1 is split_qkv + apply_rope
 * (decoder_compiler.cpp:96-148) writing q, k and that vt from the fp32 QKV rows. */
int64_t sfg_hip_attn_vt_ld_v1(int64_t seq_kv);
int sfg_hip_qkv_split_rope_vt_v1(const float* qkv, const float* rope_table, int64_t batch,
                                 int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                 uint16_t* q, uint16_t* k, uint16_t* vt, int64_t ld_vt,
                                 void* stream);
int sfg_hip_attn_prefill_vt_v1(const uint16_t* q, const uint16_t* k, const uint16_t* vt,
                               int64_t ld_vt, void* out, int out_dtype, int64_t batch,
                               int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_kv,
                               int64_t head_dim, int causal, float scale, void* stream);

/* Paged Split-KV decode (attention_compiler.cpp:244-285 split/merge,
 * next_milestones.cpp:137-184 page walk).  q fp32 [B][Hq][D] (one new token per
 * sequence), pools bf16: K [num_pages][Hkv][page_tokens][D], V
 * [num_pages][Hkv][D][page_tokens]; page_table
 * [B][pages_per_seq], seq_lens[B] (each <= pages_per_seq*page_tokens).  out
 * merged [B][Hq*D] in out_dtype.  Any head_dim up to 256 and any page size:
 * head_dim 128 / 64 with 16-token pages and a GQA group Hq/Hkv in
 * {1, 2, 4, 8, 16} run the MFMA split kernel, everything else the row kernel
 * of sfg_hip_attn_paged_v1.  kv_splits <= 0 picks a split count.  Page ids
 * are validated on the host against num_pages only when validate_pages != 0
 * (this reads the table back and synchronises the stream). */
size_t sfg_hip_attn_decode_workspace_v1(int64_t batch, int64_t q_heads, int64_t head_dim,
                                        int64_t max_context, int64_t page_tokens,
                                        int32_t kv_splits);
int sfg_hip_attn_decode_paged_v1(const float* q, const uint16_t* k_pool,
                                 const uint16_t* v_pool, const int32_t* page_table,
                                 const int32_t* seq_lens, void* out, int out_dtype,
                                 int64_t batch, int64_t q_heads, int64_t kv_heads,
                                 int64_t head_dim, int64_t page_tokens, int64_t pages_per_seq,
                                 int64_t num_pages, int64_t max_context, int32_t kv_splits,
                                 float scale, int validate_pages, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* The same paged Split-KV decode with no workspace argument and no allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory or pass a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The split partials live in
 * a library-held device array of SFG_DECODE_SCRATCH_BYTES (16 MiB) per device,
 * resident from the first call on a device until the process ends; a call
 * whose partials, batch * q_heads * splits * (head_dim + 2) * 4 bytes (each
 * part rounded up to 256), exceed it returns SFG_ERR_WORKSPACE.  Every call on
 * one device shares that device's array: calls that overlap on one GPU (other
 * streams, other host threads) race and must be serialised by the caller.
 * Nothing in the array needs clearing: each call writes every partial before
 * reading it.  Page ids outside [0, num_pages) are skipped on the device (no
 * host-side table validation: it would synchronise the stream).  Results are
 * bit-identical to sfg_hip_attn_decode_paged_v1 with the same split count.
 * Under graph capture: make the first call on each device outside the
 * capture (it looks the array's address up with hipGetSymbolAddress, which
 * may load the code object); a captured call records only kernel launches,
 * no memset or copy.  Every replay of every captured call on one device uses
 * the same array, so replays on different streams race like eager calls. */
#define SFG_DECODE_SCRATCH_BYTES ((size_t)16 << 20)
int sfg_hip_attn_decode_paged_noalloc_v1(const float* q, const uint16_t* k_pool,
                                         const uint16_t* v_pool, const int32_t* page_table,
                                         const int32_t* seq_lens, void* out, int out_dtype,
                                         int64_t batch, int64_t q_heads, int64_t kv_heads,
                                         int64_t head_dim, int64_t page_tokens,
                                         int64_t pages_per_seq, int64_t num_pages,
                                         int64_t max_context, int32_t kv_splits, float scale,
                                         void* stream);

/* Paged attention in general: execute_paged_decode_attention /
 * execute_decode_attention (next_milestones.cpp:583-609, attention_compiler.cpp:
 * 923-1007) for seq_q >= 1 new query rows per sequence, any head_dim up to 256,
 * any page size, pools of kv_dtype SFG_F32 or SFG_BF16 (layouts as above).
 * q fp32 and out (out_dtype) are head-major [B][Hq][seq_q][D], the reference's
 * AttentionData layout.  Sequence b attends over its first L_b keys, L_b =
 * seq_lens[b] (device) or max_context when seq_lens is NULL; with causal != 0
 * query row i sees key j iff j <= L_b - seq_q + i (attention_compiler.cpp:68-72),
 * so seq_q = 1 sees all of them.  A row with no visible key comes out NaN, as
 * the reference's 0 / 0.  The MFMA split kernel takes the shapes it lowers
 * (bf16, head_dim 64 / 128, 16-token pages, one row, GQA group up to 16);
 * the rest run one wave per (sequence, row, head, split) with fp32 dot
 * products over the head dimension and an fp32 online softmax.  Errors:
 * SFG_ERR_INVALID_CONFIG for causal with seq_q > max_context (validate_config,
 * attention_compiler.cpp:23-29), SFG_ERR_UNSUPPORTED for head_dim > 256. */
size_t sfg_hip_attn_paged_workspace_v1(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                       int64_t seq_q, int64_t head_dim, int kv_dtype,
                                       int64_t max_context, int64_t page_tokens,
                                       int32_t kv_splits);
int sfg_hip_attn_paged_v1(const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                          const int32_t* page_table, const int32_t* seq_lens, void* out,
                          int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                          int64_t seq_q, int64_t head_dim, int64_t page_tokens,
                          int64_t pages_per_seq, int64_t num_pages, int64_t max_context,
                          int causal, int32_t kv_splits, float scale, int validate_pages,
                          void* workspace, size_t workspace_bytes, void* stream);

/* append_paged_kv (next_milestones.cpp:486-524) on the device pools: keys / values
 * [B][Hkv][tokens][D] (dtype SFG_F32 or SFG_BF16) are stored in the pools' dtype
 * (pool_dtype SFG_F32 or SFG_BF16; the _paged_v1 form takes bf16 pools) at token
 * positions start_b + t, start_b = seq_lens[b] (device) when seq_lens != NULL,
 * else `start`, through page_table [B][pages_per_seq] into
 * K [num_pages][Hkv][page_tokens][D] / V [num_pages][Hkv][D][page_tokens].  Pages
 * are assigned by the caller (the host allocator, as the reference's free list);
 * positions past the table's capacity and page ids outside [0, num_pages) are
 * not written.  advance != 0 adds `tokens` to seq_lens afterwards.  Any
 * head_dim and page size.
 * gather_paged_kv (next_milestones.cpp:554-581): the first `length` tokens of every
 * sequence back to keys / values [B][Hkv][length][D] fp32. */
int sfg_hip_kv_append_pool_v1(const void* keys, const void* values, int dtype, void* k_pool,
                              void* v_pool, int pool_dtype, const int32_t* page_table,
                              int32_t* seq_lens, int64_t start, int advance, int64_t batch,
                              int64_t kv_heads, int64_t tokens, int64_t head_dim, int64_t page_tokens,
                              int64_t pages_per_seq, int64_t num_pages, void* stream);
int sfg_hip_kv_gather_pool_v1(const void* k_pool, const void* v_pool, int pool_dtype,
                              const int32_t* page_table, int64_t batch, int64_t kv_heads,
                              int64_t length, int64_t head_dim, int64_t page_tokens,
                              int64_t pages_per_seq, int64_t num_pages, float* keys, float* values,
                              void* stream);
int sfg_hip_kv_append_paged_v1(const void* keys, const void* values, int dtype, uint16_t* k_pool,
                               uint16_t* v_pool, const int32_t* page_table, int32_t* seq_lens,
                               int64_t start, int advance, int64_t batch, int64_t kv_heads,
                               int64_t tokens, int64_t head_dim, int64_t page_tokens,
                               int64_t pages_per_seq, int64_t num_pages, void* stream);
int sfg_hip_kv_gather_paged_v1(const uint16_t* k_pool, const uint16_t* v_pool,
                               const int32_t* page_table, int64_t batch, int64_t kv_heads,
                               int64_t length, int64_t head_dim, int64_t page_tokens,
                               int64_t pages_per_seq, int64_t num_pages, float* keys, float* values,
                               void* stream);

/* MoE routing: Router -> Softmax -> TopK -> Histogram -> PrefixSum -> Dispatch
 * (route_topk, moe_compiler.cpp:412-455; dispatch_tokens, 496-528).
 * x fp32 [T][H], router fp32 [H][E], bias fp32 [E] or NULL.  Logits are
 * sequential fp32 FMA chains over H (bit-identical to the oracle); top-k by
 * logit, ties to the lower expert index.  Outputs (device, int32 / fp32):
 * ids/weights [T][k]; counts [E]; offsets [E+1]; token_ids, route_slots,
 * routing_weights [T*k] in expert-major, token-ascending order; and
 * position [T][k] = index of each (token, slot) in that order. */
size_t sfg_hip_moe_route_workspace_v1(int64_t tokens, int64_t experts, int64_t top_k);
int sfg_hip_moe_route_v1(const float* x, const float* router, const float* bias,
                         int64_t tokens, int64_t hidden, int64_t experts, int64_t top_k,
                         int32_t* ids, float* weights, int32_t* counts, int32_t* offsets,
                         int32_t* token_ids, int32_t* route_slots, float* routing_weights,
                         int32_t* position, void* workspace, size_t workspace_bytes,
                         void* stream);
/* Same pipeline from a given routing trace (decoder_compiler.cpp:281-284).  An
 * expert id outside [0, experts) (the reference refuses one,
 * next_milestones.cpp:427-428) is left out of counts, offsets and the segments,
 * and its position is -1: sfg_hip_moe_combine_v1 adds nothing for it. */
int sfg_hip_moe_dispatch_trace_v1(const int32_t* ids, const float* weights, int64_t tokens,
                                  int64_t experts, int64_t top_k, int32_t* counts,
                                  int32_t* offsets, int32_t* token_ids, int32_t* route_slots,
                                  float* routing_weights, int32_t* position, void* stream);

/* Variable-M grouped expert GEMMs (compute_task, moe_compiler.cpp:121-155):
 * stage 1: act[r] = (x[tok(r)] W1[e]) * silu(x[tok(r)] W3[e]) for dispatched rows r
 *          of expert e = segment(r); w13 [E][2I][H] (rows [0,I) W1^T, [I,2I) W3^T),
 *          x bf16 [T][H], act bf16 [T*k][I];
 * stage 2: y[r] = act[r] W2[e], w2 [E][H][I], y fp32 [T*k][H].
 * w dtype SFG_BF16 or SFG_I8 (+ scales [E][2I] / [E][H]). */
/* Workspace bytes sfg_hip_moe_experts_v1 needs for these sizes.  It is 0 for
 * every shape this build lowers (both stages write only act and y); the query
 * keeps the workspace convention of the other entries, so a caller that sizes
 * and passes what it returns stays correct if a later kernel needs scratch. */
size_t sfg_hip_moe_expert_workspace_v1(int64_t tokens, int64_t hidden, int64_t inter,
                                       int64_t experts, int64_t top_k);
int sfg_hip_moe_experts_v1(const uint16_t* x, const int32_t* offsets, const int32_t* token_ids,
                           const void* w13, const float* s13, const void* w2, const float* s2,
                           int w_dtype, int w_layout, uint16_t* act, float* y, int64_t tokens,
                           int64_t hidden, int64_t inter, int64_t experts, int64_t top_k,
                           void* workspace, size_t workspace_bytes, void* stream);
/* Weighted combine (moe_compiler.cpp:219-226) fused with the FFN residual
 * (decoder_compiler.cpp:277): out[t] = residual[t] + sum_s w[t][s] * y[position[t][s]]. */
int sfg_hip_moe_combine_v1(const float* y, const int32_t* position, const float* weights,
                           const float* residual, float* out, int64_t tokens, int64_t hidden,
                           int64_t top_k, void* stream);

/* ---------------- whole layer: execute_once (decoder_compiler.cpp:218-304) ---------------- */

typedef struct {
    int32_t abi;  /* SFG_HIP_ABI_VERSION */
    int32_t batch, sequence, hidden, intermediate, query_heads, kv_heads, head_dim;
    float rms_epsilon, rope_theta;
    int32_t causal;
    int32_t ffn;        /* 0 dense SwiGLU, 1 MoE */
    int32_t experts, top_k;
    int32_t context;    /* 0: prefill; > 0: decode step of `sequence` new tokens per
                         * sequence over this many cached tokens (causal: new token i
                         * sees cached key j iff j <= context - sequence + i) */
    int32_t page_tokens, pages_per_seq, num_pages;
    int32_t act_dtype;  /* SFG_F32 (all-fp32 path) or SFG_BF16 */
    int32_t weight_dtype; /* SFG_F32, SFG_BF16 or SFG_I8 */
    int32_t kv_splits;  /* decode; <= 0: automatic */
    int32_t use_routing_trace;
    int32_t weight_layout; /* layout of every projection / expert weight */
    int32_t kv_append;  /* decode only.  0: the reference's semantics -- RoPE at position 0
                         * within the step, the step's K/V computed and discarded
                         * (decoder_compiler.cpp:96-104, 238-243).  1: RoPE at the
                         * sequence's true position (its cached length), the step's
                         * K/V written into the pools at that position (append_paged_kv,
                         * next_milestones.cpp:486-524; the page must already be in the
                         * table) and attention over the cache including it.  Not a
                         * reference mode: its outputs differ from execute_once's.
                         * Needs a capacity-sized rope_table (below).  A sequence already
                         * at capacity (pages_per_seq * page_tokens) gets nothing
                         * appended and its length stays at the capacity: the caller
                         * must refuse such a step, as the reference's append_paged_kv
                         * does ("paged KV capacity exceeded"). */
    int32_t gemm_tile;  /* sfg_gemm_tile of the prefill projection / expert GEMMs;
                         * SFG_TILE_AUTO (0) picks per shape.  Same results for every
                         * tile; a plan-policy knob searched by the plan optimiser. */
    int32_t attn_waves; /* bf16 flash prefill (head_dim 128): 4 or 8 waves, i.e. 128 or
                         * 256 query rows per workgroup; 0: 8 when the 256-row grid
                         * holds at least 4 workgroups per CU, else 4.  Same results
                         * either way. */
} sfg_layer_desc;

typedef struct {
    const float* rms1; const float* rms2;        /* [H] */
    const void* w_qkv; const float* s_qkv;       /* [H + 2 Hkv D][H] */
    const void* w_o; const float* s_o;           /* [H][H] */
    const void* w_gate_up; const float* s_gate_up; /* dense: [2I][H] */
    const void* w_down; const float* s_down;     /* dense: [H][I] */
    const float* router; const float* router_bias; /* MoE: [H][E], [E] or NULL */
    const void* w13; const float* s13;           /* MoE: [E][2I][H] */
    const void* w2; const float* s2;             /* MoE: [E][H][I] */
    void* k_pool; void* v_pool;                  /* decode: paged pools in the activation dtype
                                                  * (bf16, or fp32 on the fp32 path); written
                                                  * when kv_append */
    const int32_t* page_table;                   /* decode: [B][pages_per_seq] */
    const float* rope_table;                     /* [rows][D/2][2] device copy of
                                                  * sfg_hip_rope_table_host_v1 with rows =
                                                  * S (prefill, and decode: positions 0..S-1
                                                  * within the step), or pages_per_seq *
                                                  * page_tokens when kv_append: the new
                                                  * tokens rotate at their true positions,
                                                  * clamped to capacity - 1.  May be NULL
                                                  * when head_dim < 2 (nothing rotates) */
} sfg_layer_weights;

/* Stage marks recorded into caller-created events when io->stage_events != NULL. */
enum sfg_stage_mark {
    SFG_MARK_START = 0, SFG_MARK_NORM1, SFG_MARK_QKV, SFG_MARK_ROPE, SFG_MARK_ATTN_MAIN,
    SFG_MARK_ATTN, SFG_MARK_OPROJ, SFG_MARK_NORM2, SFG_MARK_ROUTE, SFG_MARK_FFN_UP,
    SFG_MARK_FFN_DOWN, SFG_MARK_END, SFG_NUM_MARKS
};

typedef struct {
    const float* x;                  /* [rows][H] fp32 */
    float* out;                      /* [rows][H] fp32 */
    const int32_t* trace_ids;        /* optional routing trace [rows][k] */
    const float* trace_weights;
    void** stage_events;             /* NULL or SFG_NUM_MARKS hipEvent_t */
    int32_t* seq_lens;               /* kv_append: device [B] cached lengths, advanced by one
                                      * after the step; NULL: every sequence holds `context` */
} sfg_layer_io;

size_t sfg_hip_decoder_layer_workspace_v1(const sfg_layer_desc* desc);

/* Stage intermediates a layer call leaves in its workspace, for stage-level
 * validation: execute_once's own intermediate buffers (decoder_compiler.cpp:
 * 218-304 -- merged attention, the residual r1, the second RMSNorm's output and
 * the routing of route_topk, moe_compiler.cpp:412-455).  After a call returns
 * (once its stream has drained), bytes [offset, offset + bytes) of the same
 * workspace hold the tap for the same descriptor:
 *   SFG_TAP_ATTN          merged attention [rows][H], act dtype
 *   SFG_TAP_RESIDUAL1     r1 = attn Wo + x, [rows][H] fp32
 *   SFG_TAP_NORM2         RMSNorm(r1) * rms2, [rows][H] act dtype
 *   SFG_TAP_ROUTE_INPUT   the router's fp32 input RMSNorm(r1) * rms2 [rows][H] (MoE)
 *   SFG_TAP_ROUTE_IDS     top-k expert ids [rows][k] int32     } MoE routed on
 *   SFG_TAP_ROUTE_WEIGHTS renormalised weights [rows][k] fp32  } the device only
 * dtype receives an sfg_dtype.  No reference entry point exposes these; the
 * reference's tests compare whole-layer outputs only. */
enum sfg_layer_tap {
    SFG_TAP_ATTN = 0, SFG_TAP_RESIDUAL1, SFG_TAP_NORM2, SFG_TAP_ROUTE_INPUT, SFG_TAP_ROUTE_IDS,
    SFG_TAP_ROUTE_WEIGHTS, SFG_NUM_TAPS
};
int sfg_hip_decoder_layer_tap_v1(const sfg_layer_desc* desc, int tap, size_t* offset,
                                 size_t* bytes, int* dtype);
int sfg_hip_decoder_layer_v1(const sfg_layer_desc* desc, const sfg_layer_weights* weights,
                             const sfg_layer_io* io, void* workspace, size_t workspace_bytes,
                             void* stream);

/* ---------------- event helpers (for stage timing from any host language) ---------------- */
int sfg_hip_events_create_v1(int count, void** events);
int sfg_hip_events_destroy_v1(int count, void** events);
int sfg_hip_event_elapsed_v1(void* start, void* end, float* milliseconds);
int sfg_hip_stream_synchronize_v1(void* stream);

#ifdef __cplusplus
}
#endif
#endif
