// sfg_kernels.hpp -- launchers shared between the kernel translation units and
// the C-ABI layer (sfg_api.hip).  Launchers assume arguments were validated by
// the ABI layer; they never allocate.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/sfg_hip.h"
#include "sfg_device.hpp"

namespace sfg {

// elementwise
// y32 (optional): the same normalised rows also written as fp32.
void launch_rmsnorm(const float* x, const float* w, void* y, int y_dtype, int64_t rows,
                    int64_t width, float eps, hipStream_t stream, float* y32 = nullptr);
void launch_split_rope(const float* qkv, const float* table, int64_t batch, int64_t seq,
                       int64_t q_heads, int64_t kv_heads, int64_t head_dim, void* q, void* k,
                       void* v, int out_dtype, hipStream_t stream);
void launch_pack_weight(const float* src, int64_t k, int64_t n, int64_t ld, void* dst,
                        int dtype, int layout, hipStream_t stream);
void launch_quantize_weight(const float* src, int64_t k, int64_t n, int8_t* dst, float* scales,
                            int layout, hipStream_t stream);
void launch_to_bf16(const float* src, uint16_t* dst, int64_t count, hipStream_t stream);
void launch_fill_zero(void* dst, size_t bytes, hipStream_t stream);

// QKV-projection epilogue of the bf16 prefill (kEpiQkvRope): RoPE'd Q / K as
// [B][H*][S][128] bf16 and V^T [B][Hkv][128][ld_vt] bf16, the product itself
// never stored.  Needs the direct-to-LDS GEMM path (gemm_qkv_rope_supported).
constexpr int kEpiQkvRope = 16;
struct QkvRopeOut {
    const float2* rope;          // [S][64] (cos, sin)
    int64_t seq; int q_heads, kv_heads;
    uint16_t* q; uint16_t* k; uint16_t* vt; int64_t ld_vt;
};

// GEMM family.  A grouped problem: `groups` independent products sharing N, K;
// group g covers rows [row_begin(g), row_end(g)) of the (virtual) row space,
// given by `offsets` (device, groups+1 entries) or a single dense group.  A's
// row r is read from a_rows[r] when a_rows != nullptr (dispatch gather).
struct GemmProblem {
    const void* a; int a_dtype; int64_t lda;
    const int32_t* a_rows;      // optional gather (row indices into A)
    int64_t a_rows_limit;       // rows of A addressable through a_rows
    const void* b; int b_dtype; int64_t ldb; const float* b_scales;
    int64_t b_group_stride;     // elements between groups' B matrices
    int64_t s_group_stride;     // scales between groups
    void* c; int c_dtype; int64_t ldc;
    const float* residual; int64_t ldr;
    int64_t m, n, k;            // m: total rows (dense) or upper bound (grouped)
    int epilogue;
    int b_layout;               // SFG_LAYOUT_NK or SFG_LAYOUT_TILED
    const int32_t* offsets;     // grouped: device [groups+1]; nullptr = dense
    int groups;
    QkvRopeOut qkv;             // epilogue kEpiQkvRope only
    int tile;                   // sfg_gemm_tile of the direct-to-LDS path (0: by shape)
    int xcds;                   // XCDs workgroups are dealt over (launch_gemm fills it)
};

// XCDs of the device that owns `stream` (hipDeviceAttributeNumberOfXccs),
// queried once per device: the dispatcher deals consecutive workgroup ids over
// them in turn, which the XCD-aware tile orders undo.
int device_xcds(hipStream_t stream);
// Compute units of the stream's device (cached per device).
int device_cus(hipStream_t stream);

bool gemm_qkv_rope_supported(const GemmProblem& p);
size_t gemm_workspace_bytes(int64_t m, int64_t n, int64_t k);
// The layout launch_gemm reads fastest for these rows (see sfg_layout).
int gemm_preferred_layout(int64_t rows, int64_t k, bool grouped);
// Returns SFG_OK or an error code (unsupported combination).
int launch_gemm(const GemmProblem& p, void* workspace, size_t workspace_bytes,
                hipStream_t stream);

// attention
// Row-per-wave online softmax, head_dim <= 256 (SFG_ERR_UNSUPPORTED beyond).
int launch_attn_prefill_f32(const float* q, const float* k, const float* v, void* out,
                             int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                             int64_t seq_q, int64_t seq_kv, int64_t head_dim, int causal,
                             float scale, hipStream_t stream);
// MFMA flash prefill at head_dim 64 / 128; other head dims up to 256 run the
// row-per-wave kernel on the bf16 operands.
int launch_attn_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, void* out,
                             int out_dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                             int64_t seq_q, int64_t seq_kv, int64_t head_dim, int causal,
                             float scale, hipStream_t stream);
// Flash prefill over V^T [B][Hkv][128][ld_vt] (keys >= seq_kv zero); ld_vt is
// attn_vt_ld(seq_kv).  waves: 4 or 8 waves (128 / 256 query rows) per
// workgroup; anything else means 4.  launch_v_transpose writes that V^T from fp32 QKV rows.
int64_t attn_vt_ld(int64_t seq_kv);
int launch_attn_prefill_vt(const uint16_t* q, const uint16_t* k, const uint16_t* vt, int64_t ld_vt,
                           void* out, int out_dtype, int64_t batch, int64_t q_heads,
                           int64_t kv_heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                           int causal, float scale, int waves, hipStream_t stream);
void launch_v_transpose(const float* qkv, int64_t batch, int64_t seq, int64_t q_heads,
                        int64_t kv_heads, int64_t ld_vt, uint16_t* vt, hipStream_t stream);
int decode_split_count(int64_t batch, int64_t kv_heads, int64_t max_context,
                       int64_t page_tokens, int32_t requested);
size_t decode_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_dim, int splits);
// The MFMA split-KV decode: bf16 pools, head_dim 64 / 128, 16-token pages, one
// new token per sequence, GQA group 1 / 2 / 4 / 8 / 16 (decode_mfma_supported);
// SFG_ERR_UNSUPPORTED otherwise (launch_attn_paged_rows takes those).
bool decode_mfma_supported(int kv_dtype, int64_t head_dim, int64_t page_tokens, int64_t group,
                           int64_t seq_q);
int launch_attn_decode_paged(const float* q, int64_t q_row_stride, const float* rope, int rope_pos,
                             const uint16_t* k_pool, const uint16_t* v_pool,
                             const int32_t* page_table, const int32_t* seq_lens, int64_t max_context,
                             int len_extra, void* out, int out_dtype, int64_t batch, int64_t q_heads,
                             int64_t kv_heads, int64_t head_dim, int64_t page_tokens,
                             int64_t pages_per_seq, int64_t num_pages, int splits, float scale,
                             void* workspace, hipStream_t stream, hipEvent_t mid_event);

// Generic paged attention (any head_dim <= 256, any page size, seq_q >= 1 rows
// per sequence under the causal offset, fp32 or bf16 pools).  Q (fp32) and the
// output are addressed by element strides of (batch, row, head), dims
// contiguous.  Partials of splits > 1 go to the workspace
// (paged_rows_workspace_bytes(B seq_q Hq, D, splits)).
struct PagedRowsLaunch {
    const float* q; int64_t q_stride_b, q_stride_i, q_stride_h;
    const float* rope; int rope_rows; int rope_pos;  // optional RoPE of Q (rope_pos < 0: at seq_lens[b] + i)
    const void* k_pool; const void* v_pool; int kv_dtype;
    const int32_t* page_table; const int32_t* seq_lens;
    int64_t max_context; int len_extra;     // keys per sequence: (seq_lens[b] or max_context) + len_extra
    void* out; int out_dtype; int64_t out_stride_b, out_stride_i, out_stride_h;
    int64_t batch, q_heads, kv_heads, seq_q, head_dim, page_tokens, pages_per_seq, num_pages;
    int splits, causal; float scale;
    hipEvent_t mid_event;                   // recorded between the split and combine kernels
};
int paged_rows_split_count(int64_t rows, int64_t max_keys, int32_t requested);
size_t paged_rows_workspace_bytes(int64_t rows, int64_t head_dim, int splits);
int launch_attn_paged_rows(const PagedRowsLaunch& a, void* workspace, hipStream_t stream);

// Paged KV append / gather (pages pre-assigned in the tables), any head_dim and
// page size, pools fp32 or bf16.  Sources are [b][h][t][D] with element
// strides sb / sh / st; rope (optional) rotates the keys at their positions;
// advance != 0 adds `tokens` to seq_lens afterwards.
int launch_kv_append(const void* keys, const void* values, int src_dtype, int64_t sb, int64_t sh,
                     int64_t st, const float* rope, void* k_pool, void* v_pool, int pool_dtype,
                     const int32_t* page_table, int32_t* seq_lens, int64_t start, int advance,
                     int64_t batch, int64_t kv_heads, int64_t tokens, int64_t head_dim,
                     int64_t page_tokens, int64_t pages_per_seq, int64_t num_pages,
                     hipStream_t stream);
void launch_kv_advance(int32_t* seq_lens, int64_t batch, int64_t tokens, int64_t capacity,
                       hipStream_t stream);
int launch_kv_gather(const void* k_pool, const void* v_pool, int pool_dtype, const int32_t* page_table,
                     int64_t batch, int64_t kv_heads, int64_t length, int64_t head_dim,
                     int64_t page_tokens, int64_t pages_per_seq, int64_t num_pages, float* keys,
                     float* values, hipStream_t stream);

// MoE
size_t moe_route_workspace_bytes(int64_t tokens, int64_t experts, int64_t top_k);
int launch_moe_router(const float* x, const float* router, const float* bias, int64_t tokens,
                      int64_t hidden, int64_t experts, int64_t top_k, int32_t* ids,
                      float* weights, hipStream_t stream);
int launch_moe_dispatch(const int32_t* ids, const float* weights, int64_t tokens,
                        int64_t experts, int64_t top_k, int32_t* counts, int32_t* offsets,
                        int32_t* token_ids, int32_t* route_slots, float* routing_weights,
                        int32_t* position, hipStream_t stream);
void launch_moe_combine(const float* y, const int32_t* position, const float* weights,
                        const float* residual, float* out, int64_t tokens, int64_t hidden,
                        int64_t top_k, hipStream_t stream);

}  // namespace sfg
